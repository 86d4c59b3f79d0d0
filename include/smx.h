/*
 * smx.h - C ABI of the MI355X (gfx950) batch-1 Q4_0 decode path.
 *
 * Every entry point:
 *   - takes the HIP stream as an opaque `void*` first (NULL = the default
 *     stream), then raw device pointers and integer sizes;
 *   - validates its arguments on the host before touching the GPU and
 *     returns SMX_EINVAL (with a message from smx_last_error()) when they are
 *     wrong, so a bad call never reaches a kernel;
 *   - otherwise enqueues its kernels on `stream` and returns 0, or the
 *     hipError_t value reported by the launch;
 *   - never allocates, never synchronises, never throws across the ABI, and
 *     is safe to record into a HIP graph.
 *
 * The reference's only native C ABI on this path is
 *   extern "C" void launch_head_q6s(void* stream, uint8_t* x, uint8_t* w,
 *                                   uint8_t* y, int rows, int decode)
 * (src/spark_vllm_ascend/native/head/head_q6.asc:35, declared at
 * src/spark_vllm_ascend/native/head/extension.cpp:6) plus the argument checks
 * of its TORCH_CHECK wrapper (extension.cpp:8-10).  The rest of the
 * reference's decode path is one DSL megakernel (kernels/layer.py:48-109);
 * each function below replaces one of its stages and cites it.
 *
 * Tensor formats (all row-major, contiguous):
 *   bf16   : uint16 bit patterns of bfloat16.
 *   Q4_0   : GGUF ggml type 2.  A row of k weights is k/32 blocks of 18
 *            bytes: fp16 little-endian scale d, then 16 bytes qs; element
 *            j<16 is (qs[j] & 15) - 8, element j>=16 is (qs[j-16] >> 4) - 8,
 *            value = d * element.
 *   KV cache: [num_blocks, block_size, num_kv_heads, head_dim] bf16, one
 *            tensor for K and one for V (vLLM's paged layout).
 */
#ifndef SMX_H
#define SMX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SMX_ABI_VERSION 10

/* Return codes besides 0 and hipError_t values. */
#define SMX_EINVAL 10001      /* an argument failed validation */
#define SMX_EUNSUPPORTED 10002 /* a valid shape the library has no kernel for */

/* ABI version of the loaded library (SMX_ABI_VERSION it was built with). */
int smx_abi_version(void);

/* Text of the last validation error raised on the calling thread. */
const char* smx_last_error(void);

/*
 * Q4_0 -> bf16 dequantisation, bit-exact: out[r, j] = RNE_bf16(float(d) * q).
 * w: n rows of k/32 Q4_0 blocks; out: [n, k] bf16.  Requires k % 32 == 0.
 * Replaces unpack_q4 + gguf dequantize + .bfloat16()
 * (src/spark_vllm_ascend/integration/weights.py:28-40,
 *  src/tools/deployment/prepare_model.py:62-64).
 */
int smx_q4_0_dequant_bf16(void* stream, const void* w, void* out,
                          int64_t n, int64_t k);

/*
 * Q4_0 dequant-fused GEMV for one activation row:
 *   y[r] = RNE_bf16( sum_b float(d_rb) * sum_j x[32b+j] * q_rbj )
 * with fp32 accumulation.  x: [k] bf16; w: [n, k/32] Q4_0 blocks;
 * y: [n] bf16.  Requires k % 32 == 0 and n >= 1.
 * Replaces GemvStage.calculate and its callers (NativeLinear.execute_o,
 * execute_down, NativeUp, FusedQkvStage: src/spark_vllm_ascend/kernels/
 * linear.py:16-200,339-370, kernels/qkv.py:201-236).
 */
int smx_q4_0_gemv(void* stream, const void* x, const void* w, void* y,
                  int64_t n, int64_t k);

/*
 * Fused gate/up Q4_0 GEMV + SwiGLU for one activation row.
 * w: [2*d, k] Q4_0 holding the gate rows [0, d) then the up rows [d, 2d)
 * (vLLM MergedColumnParallelLinear order).  out[i] =
 *   RNE_bf16( silu(g_i) * u_i ), g_i = RNE_bf16(gate GEMV), u_i likewise.
 * Replaces NativeUp.execute + activate_native
 * (src/spark_vllm_ascend/kernels/linear.py:540-611), with SwiGLU in place of
 * the reference model's GELU.
 */
int smx_q4_0_gemv_swiglu(void* stream, const void* x, const void* w,
                         void* out, int64_t d, int64_t k);

/*
 * The reference model's gate/up activation, erf-GELU through a bf16 table
 * (activate_native, src/spark_vllm_ascend/kernels/linear.py:540-577; the
 * table is built at src/spark_vllm_ascend/integration/model.py:13-16).
 * lut[SMX_GELU_LUT_ENTRIES] bf16: lut[i] = RNE_bf16(gelu(b)) for the bf16
 * bit patterns b = 0x3b00 + i (i < 2048) and b = 0xbb00 + (i - 2048) (i >=
 * 2048), gelu(x) = x * (1 + erf(x / sqrt(2))) / 2.  For the bf16 gate g:
 *   act(g) = NaN 0x7fff            g NaN or -inf
 *            g (+inf included)     g >= 128
 *            -0                    g <= -128
 *            RNE_bf16(g / 2)       |g| < 2^-9
 *            lut[index of g]       otherwise
 * and the output is RNE_bf16(act(g) * u).
 */
#define SMX_GELU_LUT_ENTRIES 4096

/* smx_q4_0_gemv_swiglu with the table GELU in place of SiLU: out[i] =
 * RNE_bf16(act(g_i) * u_i).  Replaces NativeUp.execute + activate_native
 * (src/spark_vllm_ascend/kernels/linear.py:540-611). */
int smx_q4_0_gemv_gelu(void* stream, const void* x, const void* w, const void* lut,
                       void* out, int64_t d, int64_t k);

/*
 * Q4_0 GEMV whose activation is RMSNorm(x + residual) * gamma, computed by
 * the GEMV itself (norm_ub semantics, as smx_add_rmsnorm):
 *   s = float(x) + float(residual)  (residual may be NULL)
 *   a = RNE_bf16(s / sqrt(mean(s^2) + eps) * gamma);  y = W a  (bf16)
 * and, when residual_out != NULL, residual_out = RNE_bf16(s).
 * residual_out must not alias x or residual (other workgroups still read
 * them).  k % 64 == 0, k <= 65536; x, residual, gamma, residual_out 16-byte
 * aligned, w 4-byte aligned.  Fuses the reference's add+RMSNorm with the
 * following projection (NativeUp.execute: norm_ub then the gate/up GEMV,
 * src/spark_vllm_ascend/kernels/linear.py:585-611).
 */
int smx_q4_0_add_rmsnorm_gemv(void* stream, const void* x, const void* residual,
                              const void* gamma, void* residual_out,
                              const void* w, void* y, int64_t n, int64_t k,
                              float eps);

/* smx_q4_0_add_rmsnorm_gemv followed by the SwiGLU of smx_q4_0_gemv_swiglu:
 * w is [2*d, k] (gate rows then up rows), out is [d]. */
int smx_q4_0_add_rmsnorm_gemv_swiglu(void* stream, const void* x,
                                     const void* residual, const void* gamma,
                                     void* residual_out, const void* w,
                                     void* out, int64_t d, int64_t k,
                                     float eps);

/* smx_q4_0_add_rmsnorm_gemv followed by the table GELU of
 * smx_q4_0_gemv_gelu: the whole of NativeUp.execute (norm_ub, gate/up GEMV,
 * activate_native; src/spark_vllm_ascend/kernels/linear.py:585-611). */
int smx_q4_0_add_rmsnorm_gemv_gelu(void* stream, const void* x,
                                   const void* residual, const void* gamma,
                                   void* residual_out, const void* w,
                                   const void* lut, void* out, int64_t d,
                                   int64_t k, float eps);

/*
 * smx_q4_0_add_rmsnorm_gemv for the LM head (no residual_out) that also
 * leaves greedy-argmax keys: one uint64 per workgroup in keys[num_keys],
 * reduced by smx_decode_advance.  num_keys must equal
 * smx_q4_0_argmax_keys_size(n, k) (-1 for an unsupported shape).  Replaces
 * the head GEMV + sampler pair (src/spark_vllm_ascend/integration/
 * head.py:13-16 and vLLM's greedy sampler).
 */
int64_t smx_q4_0_argmax_keys_size(int64_t n, int64_t k);
int smx_q4_0_add_rmsnorm_gemv_argmax(void* stream, const void* x,
                                     const void* residual, const void* gamma,
                                     const void* w, void* logits,
                                     uint64_t* keys, int64_t num_keys,
                                     int64_t n, int64_t k, float eps);

/*
 * Split-KV flash-decode attention, one partial per (sequence, split, q head).
 *   q: [num_seqs, n_q, head_dim] bf16
 *   k_cache, v_cache: [num_blocks, block_size, n_kv, head_dim] bf16
 *   block_table: [num_seqs, max_blocks] int32, seq_lens: [num_seqs] int32
 *   partial_o: [num_seqs, num_splits, n_q, head_dim] fp32 (normalised)
 *   partial_lse: [num_seqs, num_splits, n_q] fp32 (natural log; -inf for an
 *     empty split)
 * Split s of a sequence covers tokens [s*T, min(L, (s+1)*T)) with
 *   C = max_blocks * block_size (the block table's capacity),
 *   T = 32 * ceil(ceil(C / num_splits) / 32), L = min(seq_lens[r], C);
 * a split past L is empty (lse -inf, partial 0).  Deriving T from C rather
 * than from the device-side length lets the kernel issue its page lookups
 * before the length arrives.
 * Scores are q.k * scale in fp32; probabilities are rounded to bf16 before
 * they multiply V, and the running sum uses the unrounded fp32 values.
 * A block-table entry outside [0, num_blocks) is never dereferenced; the
 * partials of that split become NaN.
 * Supports head_dim == 128, n_q == 4 * n_kv (GQA 4:1) and power-of-two
 * block_size in [32, 4096].
 * Replaces AttentionStage (src/spark_vllm_ascend/kernels/attention.py:18-293).
 */
int smx_splitkv_decode(void* stream, const void* q, const void* k_cache,
                       const void* v_cache, const int32_t* block_table,
                       const int32_t* seq_lens, float* partial_o,
                       float* partial_lse, int32_t num_seqs,
                       int32_t num_splits, int32_t max_blocks,
                       int32_t num_blocks, int32_t block_size, int32_t n_q,
                       int32_t n_kv, int32_t head_dim, float scale);

/*
 * smx_splitkv_decode followed by smx_lse_merge on the same stream, in one
 * call: out ([num_seqs, n_q, head_dim] bf16) receives the merged attention;
 * partial_o / partial_lse are the workspace between the two launches.
 */
int smx_splitkv_decode_merged(void* stream, const void* q, const void* k_cache,
                              const void* v_cache, const int32_t* block_table,
                              const int32_t* seq_lens, float* partial_o,
                              float* partial_lse, void* out, int32_t num_seqs,
                              int32_t num_splits, int32_t max_blocks,
                              int32_t num_blocks, int32_t block_size, int32_t n_q,
                              int32_t n_kv, int32_t head_dim, float scale);

/*
 * smx_splitkv_decode_merged without caller workspace, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.
 * The split partials live in a fixed device array of SMX_NOALLOC_SCRATCH_BYTES
 * inside the library (one per GPU, held until the process ends); the call
 * allocates nothing.  It needs
 *   num_seqs * num_splits * n_q * 4 * head_dim  (rounded up to 256)
 *   + num_seqs * num_splits * n_q * 4  <=  SMX_NOALLOC_SCRATCH_BYTES
 * bytes (at n_q 32, head_dim 128: 16,512 per (sequence, split), 508 of them),
 * else SMX_EINVAL.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (two streams, concurrent graph replays) race.  The first
 * call on a device resolves the array's device address there.
 * Same arguments and result as smx_splitkv_decode_merged otherwise.
 */
#define SMX_NOALLOC_SCRATCH_BYTES (8u << 20)
int smx_splitkv_decode_merged_noalloc(void* stream, const void* q, const void* k_cache,
                                      const void* v_cache, const int32_t* block_table,
                                      const int32_t* seq_lens, void* out, int32_t num_seqs,
                                      int32_t num_splits, int32_t max_blocks,
                                      int32_t num_blocks, int32_t block_size, int32_t n_q,
                                      int32_t n_kv, int32_t head_dim, float scale);

/*
 * smx_qknorm_rope_kv_write fused into smx_splitkv_decode_merged, for one
 * decode token per sequence: qkv is the raw QKV projection
 * [num_seqs, (n_q + 2*n_kv) * head_dim]; every workgroup applies the
 * per-head q RMSNorm (q_gamma) + neox RoPE at positions[r] to its own q
 * heads, and the workgroup whose split holds positions[r] applies the k norm
 * + RoPE to the new token, writes K/V to the cache at slot_mapping[r] and
 * uses them directly.  positions[r] must be seq_lens[r] - 1 (the decode
 * token is the last of its sequence).  Replaces the reference's fused
 * QKV-stage RoPE/KV write feeding AttentionStage
 * (src/spark_vllm_ascend/kernels/qkv.py:179-236, kernels/attention.py).
 */
int smx_qknorm_rope_splitkv_decode_merged(
    void* stream, const void* qkv, const void* q_gamma, const void* k_gamma,
    const void* cos_sin, const int64_t* positions, const int64_t* slot_mapping,
    void* k_cache, void* v_cache, const int32_t* block_table,
    const int32_t* seq_lens, float* partial_o, float* partial_lse, void* out,
    int32_t num_seqs, int32_t num_splits, int32_t max_blocks,
    int32_t num_blocks, int32_t block_size, int32_t n_q, int32_t n_kv,
    int32_t head_dim, int32_t max_position, float eps, float scale);

/*
 * Per-sequence split plan for a batch of decode sequences, computed on the
 * device from the live lengths (one launch per decode step; every layer's
 * planned attention reads the same plan).  With L_r = min(seq_lens[r], C),
 * T = sum_r L_r and
 *   chunk = 128 * ceil(max(ceil(T / num_items),
 *                          ceil(max_r L_r / num_splits), 1) / 128),
 * sequence r gets n_r = ceil(L_r / chunk) <= num_splits splits; split j
 * covers tokens [j*chunk, min(L_r, (j+1)*chunk)).  The splits are numbered
 * sequence by sequence and described by plan records (a record per split,
 * unused records past the last one), at most num_items + num_seqs of them:
 *   plan: [num_items + num_seqs, SMX_SPLITKV_PLAN_WORDS] uint32
 *   partial_o [num_seqs, num_splits, n_q, head_dim] fp32 (16-byte aligned),
 *   partial_lse [num_seqs, num_splits, n_q] fp32: the slots (r, j >= n_r),
 *     which no split writes, are set to 0 / -inf here, so pass the same
 *     buffers to the planned attention calls that use this plan.
 * positions / slot_mapping ([num_seqs] int64) may be NULL unless the plan
 * feeds smx_qknorm_rope_splitkv_decode_planned_merged; when both are given,
 * every record's word 3 carries bit 31 (SMX_SPLITKV_PLAN_HAS_POSITIONS)
 * above the split index.  num_seqs <= 64.
 * Counterpart of execute_serial's device-side task list, parts =
 * ceil(length / width) from the live length (src/spark_vllm_ascend/kernels/
 * attention.py:120-128), with the splits balanced across the batch.
 */
#define SMX_SPLITKV_PLAN_WORDS 64
#define SMX_SPLITKV_PLAN_HAS_POSITIONS 0x80000000u
int smx_splitkv_plan(void* stream, const int32_t* seq_lens, const int64_t* positions,
                     const int64_t* slot_mapping, const int32_t* block_table,
                     uint32_t* plan, float* partial_o, float* partial_lse,
                     int32_t num_seqs, int32_t num_items, int32_t num_splits,
                     int32_t max_blocks, int32_t block_size, int32_t n_q,
                     int32_t head_dim);

/*
 * smx_splitkv_decode_merged over the splits of a plan (smx_splitkv_plan
 * with the same num_seqs, num_items, num_splits, block table and partial
 * buffers, enqueued earlier on the stream).  The partials are those of the
 * plan's splits, with the semantics of smx_splitkv_decode.
 */
int smx_splitkv_decode_planned_merged(
    void* stream, const void* q, const void* k_cache, const void* v_cache,
    const int32_t* block_table, const uint32_t* plan, float* partial_o,
    float* partial_lse, void* out, int32_t num_seqs, int32_t num_items,
    int32_t num_splits, int32_t max_blocks, int32_t num_blocks,
    int32_t block_size, int32_t n_q, int32_t n_kv, int32_t head_dim,
    float scale);

/*
 * smx_qknorm_rope_splitkv_decode_merged over the splits of a plan; the
 * positions and slots come from the plan.  A record without
 * SMX_SPLITKV_PLAN_HAS_POSITIONS (a plan built without positions and
 * slots) writes nothing to the cache and leaves NaN in its sequence's
 * output: the kernel cannot apply RoPE or write K/V without them.
 */
int smx_qknorm_rope_splitkv_decode_planned_merged(
    void* stream, const void* qkv, const void* q_gamma, const void* k_gamma,
    const void* cos_sin, void* k_cache, void* v_cache,
    const int32_t* block_table, const uint32_t* plan, float* partial_o,
    float* partial_lse, void* out, int32_t num_seqs, int32_t num_items,
    int32_t num_splits, int32_t max_blocks, int32_t num_blocks,
    int32_t block_size, int32_t n_q, int32_t n_kv, int32_t head_dim,
    int32_t max_position, float eps, float scale);

/*
 * Log-sum-exp merge of the split partials:
 *   w_s = exp(lse_s - max_s lse) / sum, out = RNE_bf16(sum_s w_s * o_s).
 * out: [num_seqs, n_q, head_dim] bf16.  Requires head_dim == 128.
 * Replaces merge_attention (src/spark_vllm_ascend/kernels/vector.py:45-83)
 * without the reference model's sigmoid output gate.
 */
int smx_lse_merge(void* stream, const float* partial_o,
                  const float* partial_lse, void* out, int32_t num_seqs,
                  int32_t num_splits, int32_t n_q, int32_t head_dim);

/*
 * Residual add + RMSNorm over rows of `hidden` values:
 *   s = float(x) + float(residual)            (residual may be NULL: s = x)
 *   residual_out = RNE_bf16(s)
 *   y = RNE_bf16( s * (1 / sqrt(sum(s^2)/hidden + eps)) * float(gamma) )
 * residual_out may alias residual; a NULL residual_out is not written.
 * All bf16 tensors 16-byte aligned; hidden % 8 == 0 and hidden <= 16384.
 * Replaces norm_ub / NativePool.final_norm
 * (src/spark_vllm_ascend/kernels/linear.py:202-224,299-305).
 */
int smx_add_rmsnorm(void* stream, const void* x, const void* residual,
                    const void* gamma, void* y, void* residual_out,
                    int64_t rows, int64_t hidden, float eps);

/*
 * Per-head q/k RMSNorm + neox RoPE + paged KV write, for num_tokens tokens.
 *   qkv: [num_tokens, (n_q + 2*n_kv) * head_dim] bf16 (q heads, k heads,
 *        v heads), the fused QKV GEMV output.
 *   q_gamma, k_gamma: [head_dim] bf16; eps for both norms.
 *   cos_sin: [max_position, head_dim] bf16, row p = cos(p*f_i) for
 *        i < head_dim/2 then sin(p*f_i) (vLLM cos_sin_cache layout).
 *   positions: [num_tokens] int64; slot_mapping: [num_tokens] int64
 *        (-1 = do not write this token's K/V).
 *   q_out: [num_tokens, n_q, head_dim] bf16.
 * Each norm output and each rotated value is rounded to bf16.
 * Replaces FusedQkvStage.calculate_rotated/store8 RoPE + cache write
 * (src/spark_vllm_ascend/kernels/qkv.py:179-236); the q/k norm has no
 * counterpart in the reference model.
 */
int smx_qknorm_rope_kv_write(void* stream, const void* qkv,
                             const void* q_gamma, const void* k_gamma,
                             const void* cos_sin, const int64_t* positions,
                             const int64_t* slot_mapping, void* q_out,
                             void* k_cache, void* v_cache, int32_t num_tokens,
                             int32_t n_q, int32_t n_kv, int32_t head_dim,
                             int32_t num_blocks, int32_t block_size,
                             int32_t max_position, float eps);

/*
 * SwiGLU on a [rows, 2*d] bf16 gate|up tensor: out[r, i] =
 * RNE_bf16(silu(g) * u), g = gate_up[r, i], u = gate_up[r, d + i].
 */
int smx_silu_mul(void* stream, const void* gate_up, void* out, int64_t rows,
                 int64_t d);

/*
 * The table GELU of smx_q4_0_gemv_gelu on a [rows, 2*d] bf16 gate|up
 * tensor: out[r, i] = RNE_bf16(act(g) * u), g = gate_up[r, i], u =
 * gate_up[r, d + i] (activate_native,
 * src/spark_vllm_ascend/kernels/linear.py:540-577, on a gate/up product).
 */
int smx_gelu_mul(void* stream, const void* gate_up, const void* lut, void* out,
                 int64_t rows, int64_t d);

/*
 * Embedding row gather: out[t, :] = table[ids[t], :] (bf16); an id outside
 * [0, vocab) writes a zero row.
 * Replaces VocabParallelEmbedding's lookup
 * (src/spark_vllm_ascend/plugin/spark2_5.py:320-325,362).
 */
int smx_embedding(void* stream, const void* table, const int64_t* ids,
                  void* out, int64_t num_tokens, int64_t vocab,
                  int64_t hidden);

/*
 * Greedy token: out_ids[r] = argmax_j logits[r, j] (bf16), lowest index on
 * ties, NaN counts as the largest value.  Replaces vLLM's greedy sampler at
 * temperature 0 (src/tools/benchmark/data/request.json:5).
 */
int smx_argmax_bf16(void* stream, const void* logits, int64_t rows,
                    int64_t vocab, int64_t* out_ids);

/*
 * Slot mapping of a ragged batch (vLLM's compute_slot_mapping for one KV
 * group): token t of request r (query_start_loc[r] <= t <
 * query_start_loc[r + 1], int32 [num_reqs + 1]) at positions[t] gets
 * block_table[r][p / block_size] * block_size + p % block_size; tokens past
 * the table or at negative positions get -1, and the whole padded output
 * [max_tokens] is written (entries num_tokens.. are -1).  Replaces
 * _slot_one / slot4_kernel (src/spark_vllm_ascend/integration/
 * slot_mapping.py:8-33), which covers one request per call.
 */
int smx_compute_slot_mapping(void* stream, const int32_t* query_start_loc, int32_t num_reqs,
                             const int64_t* positions, const int32_t* block_table,
                             int64_t* slot_mapping, int32_t num_tokens, int32_t max_tokens,
                             int32_t max_blocks, int32_t block_size);

/*
 * Q4_0 GEMM for m <= 16 activation rows (batched decode): y[m, n] = x[m, k]
 * W^T with W GGUF Q4_0 [n, k/32] blocks, fp32 accumulation, bf16 out;
 * k % 64 == 0, x 8-byte aligned.  The reference computes the same product
 * one token at a time (GemvStage, src/spark_vllm_ascend/kernels/
 * linear.py:16-200); the batched form is its multi-sequence extension.
 */
int smx_q4_0_gemm(void* stream, const void* x, const void* w, void* y, int64_t m, int64_t n,
                  int64_t k);

/*
 * smx_q4_0_gemm with the SwiGLU epilogue: w holds 2d rows (gate rows 0..d-1,
 * up rows d..2d-1); out[m, j] = bf16(silu(bf16(g)) * bf16(u)).  Replaces
 * NativeUp.execute + activate_native (src/spark_vllm_ascend/kernels/
 * linear.py:540-611) for several rows, with SwiGLU in place of GELU.
 */
int smx_q4_0_gemm_swiglu(void* stream, const void* x, const void* w, void* out, int64_t m,
                         int64_t d, int64_t k);

/* smx_q4_0_gemm_swiglu with the table GELU of smx_q4_0_gemv_gelu. */
int smx_q4_0_gemm_gelu(void* stream, const void* x, const void* w, const void* lut, void* out,
                       int64_t m, int64_t d, int64_t k);

/*
 * smx_q4_0_gemm (x 16-byte aligned) that also writes greedy-argmax keys:
 * keys[r][b] (b < smx_q4_0_gemm_keys_per_row(n) = ceil(n / 16)) is the
 * largest (order-preserving bf16 key of y[r][o]) << 32 | (0xffffffff - o)
 * over the outputs o of 16-column group b, for smx_decode_advance's
 * argmax_keys (NaN largest, lowest index on ties).  The batched form of the
 * head GEMV + greedy sampling (src/spark_vllm_ascend/integration/
 * head.py:12-16 and the stock argmax), without a separate argmax launch.
 */
int64_t smx_q4_0_gemm_keys_per_row(int64_t n);
int smx_q4_0_gemm_argmax(void* stream, const void* x, const void* w, void* y, uint64_t* keys,
                         int64_t m, int64_t n, int64_t k);

/*
 * Packed Q4_0 layout for the GEMMs above: the same codes and fp16 scales as
 * the GGUF blocks (lossless), moved so that each lane of a wave loads its
 * MFMA operands directly.  Per row group (16 rows; gated: 8 gate rows then
 * the 8 matching up rows) and 256-k chunk, 2304 bytes: lane l's 16 bytes for
 * blocks 0-3 at 16 l, for blocks 4-7 at 1024 + 16 l (word i = block i, byte
 * b = codes of elements 8 (l >> 4) + b and + 4 + b, low and high nibble), then
 * row (l & 15)'s 8 fp16 scales at 2048 + 16 (l & 15).  Groups past the last
 * row repeat it.  The reference repacks its Q4_0 weights into its own
 * kernel's tile layout at load time (pack, src/spark_vllm_ascend/
 * integration/weights.py:42-54, cached per layer by packed(), integration/
 * model.py:8-23, with bf16-exact scales asserted); this is the MFMA
 * counterpart, keeping the fp16 scales.
 *
 * smx_q4_0_packed_bytes: bytes of the packed form of an [n, k] matrix
 * (gated != 0: the [2d, k] gate|up matrix of the SwiGLU/GELU GEMM, n = d),
 * -1 when unsupported (k must be a positive multiple of 256).
 * smx_q4_0_repack: w (GGUF Q4_0, n rows; gated: 2n rows) -> wp, 16-byte
 * aligned, smx_q4_0_packed_bytes(n, k, gated) bytes.
 */
int64_t smx_q4_0_packed_bytes(int64_t n, int64_t k, int gated);
int smx_q4_0_repack(void* stream, const void* w, void* wp, int64_t n, int64_t k, int gated);

/*
 * smx_q4_0_gemm, smx_q4_0_gemm_swiglu, smx_q4_0_gemm_gelu and
 * smx_q4_0_gemm_argmax over packed weights (smx_q4_0_repack of the same
 * matrix, gated for the SwiGLU/GELU forms): same arguments, results equal up
 * to fp32 summation order; k % 256 == 0, x and wp 16-byte aligned.  Same
 * reference stages as the GGUF forms.
 */
int smx_q4_0_gemm_packed(void* stream, const void* x, const void* wp, void* y, int64_t m,
                         int64_t n, int64_t k);
int smx_q4_0_gemm_packed_swiglu(void* stream, const void* x, const void* wp, void* out,
                                int64_t m, int64_t d, int64_t k);
int smx_q4_0_gemm_packed_gelu(void* stream, const void* x, const void* wp, const void* lut,
                              void* out, int64_t m, int64_t d, int64_t k);
int smx_q4_0_gemm_packed_argmax(void* stream, const void* x, const void* wp, void* y,
                                uint64_t* keys, int64_t m, int64_t n, int64_t k);

/*
 * Paged KV write (vLLM reshape_and_cache): for each token t with
 * slot_mapping[t] in [0, num_blocks * block_size), copy key[t] and value[t]
 * ([n_kv, head_dim] bf16 each) into k_cache / v_cache at that slot;
 * slot -1 is skipped.  Replaces the cache stores of FusedQkvStage.store8
 * (src/spark_vllm_ascend/kernels/qkv.py:192-198,226-236).
 */
int smx_reshape_and_cache(void* stream, const void* key, const void* value,
                          void* k_cache, void* v_cache,
                          const int64_t* slot_mapping, int32_t num_tokens,
                          int32_t n_kv, int32_t head_dim, int32_t num_blocks,
                          int32_t block_size);

/*
 * Advance a decode batch by one token, on the device, so that one captured
 * graph serves every step (prompt ingestion and generation):
 *   if argmax_keys != NULL: next_ids[r] = argmax from the num_keys keys of
 *       row r written by smx_q4_0_add_rmsnorm_gemv_argmax;
 *   p = positions[r] + 1;
 *   ids[r] = forced_ids[r, p] if forced_ids != NULL and p < forced_len[r]
 *            else next_ids[r];
 *   positions[r] = p; seq_lens[r] = p + 1;
 *   slot_mapping[r] = block_table[r, p / block_size] * block_size
 *                     + p % block_size  (-1 when the table has no entry);
 *   tokens_out[r, p] = ids[r] when tokens_out != NULL and p < max_len;
 *   embed_out[r, :] = embed_table[ids[r], :] when embed_table != NULL
 *       (embed_table [vocab, hidden] bf16, zeros for an id outside [0, vocab)):
 *       the next step's embedding gather, done here instead of by a launch of
 *       its own (smx_embedding).
 * forced_ids is [rows, max_len] and forced_len an int32 [rows] device array
 * (both NULL when no tokens are forced); keeping the forced length in device
 * memory lets one graph switch from prompt to generated tokens.  The slot
 * formula is the reference's slot mapping
 * (src/spark_vllm_ascend/integration/slot_mapping.py:8-33).
 */
int smx_decode_advance(void* stream, int64_t* next_ids,
                       const uint64_t* argmax_keys, int32_t num_keys,
                       const int64_t* forced_ids, const int32_t* forced_len,
                       int64_t* ids, int64_t* positions, int32_t* seq_lens,
                       int64_t* slot_mapping, const int32_t* block_table,
                       int64_t* tokens_out, int32_t rows, int32_t max_blocks,
                       int32_t block_size, int32_t max_len,
                       const void* embed_table, void* embed_out, int64_t vocab,
                       int64_t hidden);

/*
 * Step runner: records the kernel launches that the C-ABI calls made on the
 * calling thread between smx_runner_begin and smx_runner_end would enqueue
 * (nothing is launched meanwhile; the calls still validate their arguments
 * and return their codes), then replays them as AQL kernel-dispatch packets
 * on an HSA queue of its own.  It serves the loop the reference runs as one
 * graph replay per decode step (src/spark_vllm_ascend/plugin/spark2_5.py:
 * 369-376): a step that is device-driven (positions, slots and the next
 * token advance on the device) replays `repeats` times in one call.
 *
 * code_objects: paths of this library's device code objects (one per source
 * file, built beside the library).  The runner binds to the HSA agent of the
 * current HIP device.  Recording keeps raw pointers: every buffer a recorded
 * call names must outlive the recording's replays.  A replay starts with a
 * system-scope acquire (it sees all work the host and the HIP streams have
 * completed; the caller synchronises them first) and ends with a
 * system-scope release (smx_runner_wait then makes every result visible to
 * the host).  Between two of its kernels:
 *   SMX_RUNNER_FENCES_AGENT         agent-scope acquire and release, the
 *                                   fences of a HIP stream or graph;
 *   SMX_RUNNER_FENCES_ACQUIRE_ONLY  agent-scope acquire, no release: valid
 *                                   only because every kernel of this
 *                                   library writes what a later kernel
 *                                   reads with agent-scope stores and waits
 *                                   for them before its waves end.
 * One runner per thread at a time; calls on one runner must not overlap.
 */
#define SMX_RUNNER_FENCES_AGENT 0
#define SMX_RUNNER_FENCES_ACQUIRE_ONLY 1
typedef struct smx_runner smx_runner;
int smx_runner_create(const char* const* code_objects, int32_t count, smx_runner** out);
int smx_runner_begin(smx_runner* runner);
int smx_runner_end(smx_runner* runner);
int smx_runner_num_packets(const smx_runner* runner, int64_t* out);
/* Enqueue the recorded packets `repeats` times and return; 0 or SMX_EINVAL. */
int smx_runner_replay(smx_runner* runner, int32_t repeats, int32_t fences);
/* Wait until every replay has completed, or fail after timeout_s seconds. */
int smx_runner_wait(smx_runner* runner, double timeout_s);
/* GPU time of the last replay, from its first kernel's start to its last
 * kernel's end (packet-processor timestamps), once it has completed. */
int smx_runner_elapsed(smx_runner* runner, double* seconds);
/* Waits (at most 60 s) for running replays, then frees the runner (a runner
 * whose replays do not complete in that time is left allocated).  A replay
 * that cannot write all its packets (no queue slot freed within the drain
 * timeout, 30 s unless set below) fails and breaks the runner: begin,
 * replay, wait and elapsed then fail with that reason, and destroy leaves it
 * allocated at once (the packets already written still run and read its
 * kernel arguments). */
void smx_runner_destroy(smx_runner* runner);
/* How long a replay waits for a free queue slot before it breaks the runner
 * (0..3600 s; a failure-handling test sets 0). */
int smx_runner_set_drain_timeout(smx_runner* runner, double seconds);

/* Number of nodes of a HIP graph (a hipGraph_t, e.g. a capture that has
 * ended): a recording wrapper captures the recorded function on a side
 * stream and refuses it when any launch besides this library's (which the
 * recording diverts) reached the stream.  No counterpart in the reference. */
int smx_graph_num_nodes(void* graph, int64_t* count);

#ifdef __cplusplus
}
#endif

#endif /* SMX_H */
