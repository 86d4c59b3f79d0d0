// The small fused ops around the GEMVs and attention of one decode step:
// residual add + RMSNorm, per-head q/k RMSNorm + neox RoPE + paged KV write,
// SwiGLU, embedding gather, greedy argmax and the on-device step advance.
// Each is a few kilobytes of traffic; they are written to be launch- and
// latency-cheap (one workgroup per row, vector loads, wave reductions).
#include <math.h>

#include "smx_common.h"
#include "smx_launch.h"

namespace smx {
namespace {

// Block-wide sum over the nw waves of a workgroup (wave sums, then LDS).
__device__ __forceinline__ float block_sum(float v, float* red, int nw) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  __syncthreads();
  return t;
}

// s = x + r (fp32); residual_out = bf16(s); y = bf16(s * inv_rms * gamma).
// Follows norm_ub (src/spark_vllm_ascend/kernels/linear.py:202-224): the
// normalised value uses the fp32 sum, not its bf16 rounding.  One workgroup
// per row, sized to the row (one or two 8-element chunks per thread): x, the
// residual and gamma are all loaded up front, unconditionally from clamped
// indices, so the row costs one round trip before the reduction (loads under
// a branch, or gamma loaded after the reduction, each cost another).  Each
// thread writes only the indices it read, so residual_out may alias residual.
// nt = the workgroup size (a multiple of 64), passed rather than read from
// blockDim so the kernel takes no implicit arguments.
template <int CH, bool RES>
__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* residual, const uint16_t* __restrict__ gamma,
    uint16_t* __restrict__ y, uint16_t* residual_out, int hidden, float eps, int nt) {
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const u32x4* xr = reinterpret_cast<const u32x4*>(x + row * hidden);
  const u32x4* rr = reinterpret_cast<const u32x4*>((RES ? residual : x) + row * hidden);
  const u32x4* gr = reinterpret_cast<const u32x4*>(gamma);
  const int nch = hidden / 8;
  u32x4 xa[CH], ra[CH], ga[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = min((int)threadIdx.x + c * nt, nch - 1);
    xa[c] = xr[ch];
    if constexpr (RES) ra[c] = rr[ch];
    ga[c] = gr[ch];
  }
  float sv[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool ok = (int)threadIdx.x + c * nt < nch;
    const uint32_t aw[4] = {xa[c].x, xa[c].y, xa[c].z, xa[c].w};
    const uint32_t bw[4] = {ra[c].x, ra[c].y, ra[c].z, ra[c].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[c][2 * i] = bf16_lo(aw[i]) + (RES ? bf16_lo(bw[i]) : 0.f);
      sv[c][2 * i + 1] = bf16_hi(aw[i]) + (RES ? bf16_hi(bw[i]) : 0.f);
      if (ok) ss += sv[c][2 * i] * sv[c][2 * i] + sv[c][2 * i + 1] * sv[c][2 * i + 1];
    }
  }
  ss = block_sum(ss, red, nt >> 6);
  const float inv = 1.0f / sqrtf(ss / (float)hidden + eps);
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = (int)threadIdx.x + c * nt;
    if (ch < nch) {
      const uint32_t gw[4] = {ga[c].x, ga[c].y, ga[c].z, ga[c].w};
      uint32_t yo[4], ro[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s0 = sv[c][2 * i], s1 = sv[c][2 * i + 1];
        ro[i] = pack_bf16x2(s0, s1);
        yo[i] = pack_bf16x2(s0 * inv * bf16_lo(gw[i]), s1 * inv * bf16_hi(gw[i]));
      }
      st_agent(reinterpret_cast<u32x4*>(y + row * hidden) + ch, u32x4{yo[0], yo[1], yo[2], yo[3]});
      if (residual_out)
        st_agent(reinterpret_cast<u32x4*>(residual_out + row * hidden) + ch,
                 u32x4{ro[0], ro[1], ro[2], ro[3]});
    }
  }
  stores_done();
}

// One wave per (head, token).  head_dim = 128: lane i owns dims i and i + 64,
// which are exactly a neox rotation pair.
//   q heads : RMSNorm(q_gamma) -> RoPE -> q_out
//   k heads : RMSNorm(k_gamma) -> RoPE -> k_cache[slot]
//   v heads : copy -> v_cache[slot]
// Norm outputs and rotated values are rounded to bf16 like the reference's
// stage outputs (src/spark_vllm_ascend/kernels/qkv.py:179-189).
__global__ __launch_bounds__(64) void qknorm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_gamma,
    const uint16_t* __restrict__ k_gamma, const uint16_t* __restrict__ cos_sin,
    const int64_t* __restrict__ positions, const int64_t* __restrict__ slot_mapping,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    int n_q, int n_kv, int64_t cache_slots, int max_position, float eps) {
  constexpr int HD = 128, HALF = 64;
  const int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const int nh = n_q + 2 * n_kv;
  const uint16_t* src = qkv + ((int64_t)t * nh + h) * HD;
  float a = bf16_bits_to_f32(src[lane]);
  float b = bf16_bits_to_f32(src[lane + HALF]);
  const int64_t slot = slot_mapping[t];
  const bool write_kv = slot >= 0 && slot < cache_slots;
  if (h >= n_q + n_kv) {  // v head
    if (write_kv) {
      uint16_t* dst = v_cache + (slot * n_kv + (h - n_q - n_kv)) * HD;
      st_agent(dst + lane, src[lane]);
      st_agent(dst + lane + HALF, src[lane + HALF]);
    }
    stores_done();
    return;
  }
  const uint16_t* gam = h < n_q ? q_gamma : k_gamma;
  const float ss = wave_sum(a * a + b * b);
  const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
  a = round_bf16(a * inv * bf16_bits_to_f32(gam[lane]));
  b = round_bf16(b * inv * bf16_bits_to_f32(gam[lane + HALF]));
  int64_t pos = positions[t];
  pos = pos < 0 ? 0 : (pos >= max_position ? max_position - 1 : pos);
  const uint16_t* cs = cos_sin + pos * HD;
  const float c = bf16_bits_to_f32(cs[lane]);
  const float s = bf16_bits_to_f32(cs[lane + HALF]);
  const uint16_t u = f32_to_bf16(a * c - b * s);
  const uint16_t v = f32_to_bf16(b * c + a * s);
  if (h < n_q) {
    uint16_t* dst = q_out + ((int64_t)t * n_q + h) * HD;
    st_agent(dst + lane, u);
    st_agent(dst + lane + HALF, v);
  } else if (write_kv) {
    uint16_t* dst = k_cache + (slot * n_kv + (h - n_q)) * HD;
    st_agent(dst + lane, u);
    st_agent(dst + lane + HALF, v);
  }
  stores_done();
}

// out = bf16(silu(g) * u) with silu(g) = g / (1 + exp(-g)), all in fp32.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       uint16_t* __restrict__ out, int64_t rows,
                                                       int64_t d) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256 threads per workgroup
  if (i >= rows * d) return;
  const int64_t r = i / d, c = i % d;
  const float g = bf16_bits_to_f32(gu[r * 2 * d + c]);
  const float u = bf16_bits_to_f32(gu[r * 2 * d + d + c]);
  st_agent(out + i, f32_to_bf16(g / (1.0f + expf(-g)) * u));
  stores_done();
}

// out = bf16(gelu_lut(g) * u): the reference's erf-GELU gate/up activation
// through its 4096-entry bf16 table.
__global__ __launch_bounds__(256) void gelu_mul_kernel(const uint16_t* __restrict__ gu,
                                                       const uint16_t* __restrict__ lut,
                                                       uint16_t* __restrict__ out, int64_t rows,
                                                       int64_t d) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256 threads per workgroup
  if (i >= rows * d) return;
  const int64_t r = i / d, c = i % d;
  const uint16_t g = gu[r * 2 * d + c];
  const float u = bf16_bits_to_f32(gu[r * 2 * d + d + c]);
  st_agent(out + i, f32_to_bf16(bf16_bits_to_f32(gelu_lut(g, lut)) * u));
  stores_done();
}

__global__ __launch_bounds__(256) void embedding_kernel(const uint16_t* __restrict__ table,
                                                        const int64_t* __restrict__ ids,
                                                        uint16_t* __restrict__ out, int64_t vocab,
                                                        int64_t hidden, int gx) {
  // gx workgroups of 256 threads along x (passed: no implicit arguments)
  const int64_t t = blockIdx.y;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < vocab;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < hidden; i += (int64_t)gx * 256)
    st_agent(out + t * hidden + i, ok ? table[id * hidden + i] : (uint16_t)0);
  stores_done();
}

// (value, index) ordering for argmax: larger value wins, NaN is largest,
// ties go to the lower index.
__device__ __forceinline__ bool better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

// One 1024-thread workgroup per row.
__global__ __launch_bounds__(1024) void argmax_kernel(const uint16_t* __restrict__ logits,
                                                      int64_t vocab, int64_t* __restrict__ out) {
  constexpr int64_t NT = 1024;  // threads per workgroup
  __shared__ float sv[16];
  __shared__ int64_t si[16];
  const int64_t row = blockIdx.x;
  const uint16_t* lr = logits + row * vocab;
  float bv = -INFINITY;
  int64_t bi = INT64_MAX;
  // `better` is a total order, so the scan order does not matter: 16-byte
  // chunks of 8 values, 4 chunks in flight per thread (a row is 300 KB at
  // vocab 151936), then the elements the chunks do not cover one by one.
  int64_t done = 0;
  if (((uintptr_t)lr & 15) == 0) {
    const int64_t nch = vocab >> 3;
    const u32x4* lc = reinterpret_cast<const u32x4*>(lr);
    for (int64_t c0 = threadIdx.x; c0 < nch; c0 += 4 * NT) {
      u32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t c = c0 + u * NT;
        v[u] = lc[c < nch ? c : nch - 1];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t c = c0 + u * NT;
        if (c >= nch) continue;
        const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float x = (e & 1) ? bf16_hi(w[e >> 1]) : bf16_lo(w[e >> 1]);
          if (better(x, c * 8 + e, bv, bi)) {
            bv = x;
            bi = c * 8 + e;
          }
        }
      }
    }
    done = nch << 3;
  }
  for (int64_t i = done + threadIdx.x; i < vocab; i += NT) {
    const float v = bf16_bits_to_f32(lr[i]);
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  // wave reduction with shuffles
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(bv, m, 64);
    const int64_t oi = __shfl_xor(bi, m, 64);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int wv = 1; wv < (int)(NT >> 6); ++wv)
      if (better(sv[wv], si[wv], bv, bi)) {
        bv = sv[wv];
        bi = si[wv];
      }
    st_agent(out + row, bi == INT64_MAX ? (int64_t)0 : bi);
  }
  stores_done();
}

// One workgroup of 1024 threads per row.  With argmax_keys, the row's next
// token is first reduced from the per-workgroup keys of the head GEMV
// (max value, then lowest index) and stored to next_ids.
// One 1024-thread workgroup per row, in three round trips of loads:
//  1. every thread loads 16 argmax keys at once (indices clamped to the last
//     key: a repeated key does not change a maximum), thread 0 the row's
//     position, forced length and (without keys) next id;
//  2. thread 0 loads the forced token and the block-table entry of the new
//     position (clamped indices, selected afterwards) while the keys reduce;
//  3. with embed_table, every thread gathers its share of the new token's
//     embedding row for the next step (zeros for an id outside the vocab).
__global__ __launch_bounds__(1024) void decode_advance_kernel(
    int64_t* __restrict__ next_ids, const uint64_t* __restrict__ argmax_keys, int num_keys,
    const int64_t* __restrict__ forced_ids, const int32_t* __restrict__ forced_len,
    int64_t* ids, int64_t* positions, int32_t* seq_lens, int64_t* slot_mapping,
    const int32_t* block_table, int64_t* tokens_out, int max_blocks, int block_size,
    int max_len, const uint16_t* __restrict__ embed_table, uint16_t* __restrict__ embed_out,
    int64_t vocab, int64_t hidden, int nt) {
  // nt = the workgroup size: 1024 with argmax keys or an embedding, else 64
  constexpr int KPT = 16;  // keys per thread per round trip
  __shared__ uint64_t red[16];
  __shared__ int64_t s_nid;
  const int r = blockIdx.x, tid = threadIdx.x;
  int64_t pos0 = 0, nxt0 = 0;
  int flen = 0;
  if (tid == 0) {
    pos0 = positions[r];
    if (forced_ids) flen = forced_len[r];
    if (!argmax_keys) nxt0 = next_ids[r];
  }
  uint64_t key = 0;
  if (argmax_keys) {
    const uint64_t* kr = argmax_keys + (int64_t)r * num_keys;
    for (int c0 = 0; c0 < num_keys; c0 += 1024 * KPT) {
      uint64_t kv[KPT];
#pragma unroll
      for (int j = 0; j < KPT; ++j) kv[j] = kr[min(c0 + j * 1024 + tid, num_keys - 1)];
#pragma unroll
      for (int j = 0; j < KPT; ++j) key = kv[j] > key ? kv[j] : key;
    }
  }
  int64_t p = 0, fid = 0;
  int32_t bte = 0;
  if (tid == 0) {
    p = pos0 + 1;
    if (forced_ids) fid = forced_ids[(int64_t)r * max_len + min(p, (int64_t)max_len - 1)];
    bte = block_table[(int64_t)r * max_blocks + min(p / block_size, (int64_t)max_blocks - 1)];
  }
  if (argmax_keys) {
    for (int m = 1; m < 64; m <<= 1) {
      const uint64_t o = ((uint64_t)(uint32_t)__shfl_xor((int)(key >> 32), m, 64) << 32) |
                         (uint32_t)__shfl_xor((int)(uint32_t)key, m, 64);
      key = o > key ? o : key;
    }
    if ((tid & 63) == 0) red[tid >> 6] = key;
    __syncthreads();
  }
  if (tid == 0) {
    int64_t argmax_id = nxt0;
    if (argmax_keys) {
      for (int i = 1; i < (nt >> 6); ++i) key = red[i] > key ? red[i] : key;
      argmax_id = key ? (int64_t)(0xffffffffu - (uint32_t)key) : 0;
      st_agent(next_ids + r, argmax_id);
    }
    const int64_t nid = (forced_ids && p < flen && p < max_len) ? fid : argmax_id;
    st_agent(ids + r, nid);
    st_agent(positions + r, p);
    st_agent(seq_lens + r, (int32_t)(p + 1));
    st_agent(slot_mapping + r,
             p / block_size < max_blocks ? (int64_t)bte * block_size + p % block_size : (int64_t)-1);
    if (tokens_out && p < max_len) st_agent(tokens_out + (int64_t)r * max_len + p, nid);
    s_nid = nid;
  }
  if (embed_table) {
    __syncthreads();
    const int64_t nid = s_nid;
    const bool ok = nid >= 0 && nid < vocab;
    const uint16_t* src = embed_table + (ok ? nid : 0) * hidden;
    for (int64_t i = tid; i < hidden; i += nt)
      st_agent(embed_out + (int64_t)r * hidden + i, ok ? src[i] : (uint16_t)0);
  }
  stores_done();
}

// One wave per (kv head, token): copies head_dim bf16 of K and of V.
__global__ __launch_bounds__(64) void reshape_and_cache_kernel(
    const uint16_t* __restrict__ key, const uint16_t* __restrict__ value,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const int64_t* __restrict__ slot_mapping, int n_kv, int head_dim, int64_t cache_slots) {
  const int h = blockIdx.x, t = blockIdx.y;
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= cache_slots) return;
  const int64_t src = ((int64_t)t * n_kv + h) * head_dim;
  const int64_t dst = (slot * n_kv + h) * head_dim;
  for (int i = threadIdx.x; i < head_dim; i += 64) {
    st_agent(k_cache + dst + i, key[src + i]);
    st_agent(v_cache + dst + i, value[src + i]);
  }
  stores_done();
}

// Slot of every token of a (ragged) batch: token t of request r (the r with
// query_start_loc[r] <= t < query_start_loc[r + 1]) at position p goes to
// block_table[r][p / block_size] * block_size + p % block_size; tokens in no
// request, past the block table or at a negative position get -1, and so do
// the padding entries num_tokens <= t < max_tokens.
__global__ __launch_bounds__(256) void slot_mapping_kernel(
    const int32_t* __restrict__ query_start_loc, int num_reqs,
    const int64_t* __restrict__ positions, const int32_t* __restrict__ block_table,
    int64_t* __restrict__ out, int num_tokens, int max_tokens, int max_blocks, int block_size) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= max_tokens) return;
  int64_t v = -1;
  if (t < num_tokens) {
    int lo = 0, hi = num_reqs;  // last r with query_start_loc[r] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (query_start_loc[mid] <= t) lo = mid;
      else hi = mid;
    }
    if (query_start_loc[lo] <= t && t < query_start_loc[lo + 1]) {
      const int64_t pos = positions[t];
      const int64_t blk = pos / block_size;
      if (pos >= 0 && blk < max_blocks)
        v = (int64_t)block_table[(int64_t)lo * max_blocks + blk] * block_size + pos % block_size;
    }
  }
  st_agent(out + t, v);
  stores_done();
}

}  // namespace
}  // namespace smx

#include "smx_abi_util.h"

extern "C" int smx_add_rmsnorm(void* stream, const void* x, const void* residual,
                               const void* gamma, void* y, void* residual_out, int64_t rows,
                               int64_t hidden, float eps) {
  SMX_REQUIRE(x && gamma && y, "x, gamma and y must be non-null");
  SMX_REQUIRE(rows >= 1 && rows < (1ll << 31), "rows out of range");
  SMX_REQUIRE(hidden >= 8 && hidden % 8 == 0 && hidden <= 16384,
              "hidden must be a multiple of 8 in [8, 16384]");
  SMX_REQUIRE(eps >= 0.f && isfinite(eps), "eps must be finite and >= 0");
  SMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)gamma % 16 == 0 && (uintptr_t)y % 16 == 0 &&
                  (uintptr_t)residual % 16 == 0 && (uintptr_t)residual_out % 16 == 0,
              "bf16 tensors must be 16-byte aligned");
  // one 8-element chunk per thread up to 1024 chunks (hidden 8192), else two
  const int nch = (int)(hidden / 8);
  const int threads = nch <= 1024 ? (nch + 63) / 64 * 64 : 1024;
  const auto kern = nch <= 1024 ? (residual ? smx::add_rmsnorm_kernel<1, true>
                                            : smx::add_rmsnorm_kernel<1, false>)
                                : (residual ? smx::add_rmsnorm_kernel<2, true>
                                            : smx::add_rmsnorm_kernel<2, false>);
  SMX_LAUNCH(kern, dim3((unsigned)rows), dim3(threads), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)residual, (const uint16_t*)gamma,
                     (uint16_t*)y, (uint16_t*)residual_out, (int)hidden, eps, threads);
  return (int)hipGetLastError();
}

extern "C" int smx_qknorm_rope_kv_write(void* stream, const void* qkv, const void* q_gamma,
                                        const void* k_gamma, const void* cos_sin,
                                        const int64_t* positions, const int64_t* slot_mapping,
                                        void* q_out, void* k_cache, void* v_cache,
                                        int32_t num_tokens, int32_t n_q, int32_t n_kv,
                                        int32_t head_dim, int32_t num_blocks, int32_t block_size,
                                        int32_t max_position, float eps) {
  SMX_REQUIRE(qkv && q_gamma && k_gamma && cos_sin && positions && slot_mapping && q_out &&
                  k_cache && v_cache,
              "null pointer argument");
  SMX_REQUIRE(head_dim == 128, "head_dim must be 128");
  SMX_REQUIRE(num_tokens >= 1 && num_tokens <= 65535, "num_tokens must be in [1, 65535]");
  SMX_REQUIRE(n_q >= 1 && n_kv >= 1 && n_q + 2 * n_kv <= 65535, "bad head counts");
  SMX_REQUIRE(num_blocks >= 1 && block_size >= 1 && max_position >= 1,
              "num_blocks, block_size and max_position must be >= 1");
  SMX_REQUIRE(eps >= 0.f && isfinite(eps), "eps must be finite and >= 0");
  SMX_REQUIRE((uintptr_t)positions % 8 == 0 && (uintptr_t)slot_mapping % 8 == 0,
              "int64 arrays must be 8-byte aligned");
  SMX_LAUNCH(smx::qknorm_rope_kv_kernel, dim3(n_q + 2 * n_kv, num_tokens), dim3(64), 0,
                     (hipStream_t)stream, (const uint16_t*)qkv, (const uint16_t*)q_gamma,
                     (const uint16_t*)k_gamma, (const uint16_t*)cos_sin, positions, slot_mapping,
                     (uint16_t*)q_out, (uint16_t*)k_cache, (uint16_t*)v_cache, n_q, n_kv,
                     (int64_t)num_blocks * block_size, max_position, eps);
  return (int)hipGetLastError();
}

extern "C" int smx_silu_mul(void* stream, const void* gate_up, void* out, int64_t rows,
                            int64_t d) {
  SMX_REQUIRE(gate_up && out, "null pointer argument");
  SMX_REQUIRE(rows >= 1 && d >= 1 && rows * d < (1ll << 40), "bad shape");
  const int64_t grid = (rows * d + 255) / 256;
  SMX_REQUIRE(grid < (1ll << 31), "tensor too large");
  SMX_LAUNCH(smx::silu_mul_kernel, dim3((unsigned)grid), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)gate_up, (uint16_t*)out, rows, d);
  return (int)hipGetLastError();
}

extern "C" int smx_gelu_mul(void* stream, const void* gate_up, const void* lut, void* out,
                            int64_t rows, int64_t d) {
  SMX_REQUIRE(gate_up && lut && out, "null pointer argument");
  SMX_REQUIRE((uintptr_t)gate_up % 2 == 0 && (uintptr_t)lut % 2 == 0 && (uintptr_t)out % 2 == 0,
              "gate_up, lut and out must be 2-byte aligned");
  SMX_REQUIRE(rows >= 1 && d >= 1 && rows * d < (1ll << 40), "bad shape");
  const int64_t grid = (rows * d + 255) / 256;
  SMX_REQUIRE(grid < (1ll << 31), "tensor too large");
  SMX_LAUNCH(smx::gelu_mul_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
             (const uint16_t*)gate_up, (const uint16_t*)lut, (uint16_t*)out, rows, d);
  return (int)hipGetLastError();
}

extern "C" int smx_embedding(void* stream, const void* table, const int64_t* ids, void* out,
                             int64_t num_tokens, int64_t vocab, int64_t hidden) {
  SMX_REQUIRE(table && ids && out, "null pointer argument");
  SMX_REQUIRE(num_tokens >= 1 && num_tokens <= 65535, "num_tokens must be in [1, 65535]");
  SMX_REQUIRE(vocab >= 1 && hidden >= 1, "vocab and hidden must be >= 1");
  SMX_REQUIRE((uintptr_t)ids % 8 == 0, "ids must be 8-byte aligned");
  const unsigned gx = (unsigned)((hidden + 255) / 256 < 64 ? (hidden + 255) / 256 : 64);
  SMX_LAUNCH(smx::embedding_kernel, dim3(gx, (unsigned)num_tokens), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)table, ids, (uint16_t*)out, vocab,
                     hidden, (int)gx);
  return (int)hipGetLastError();
}

extern "C" int smx_argmax_bf16(void* stream, const void* logits, int64_t rows, int64_t vocab,
                               int64_t* out_ids) {
  SMX_REQUIRE(logits && out_ids, "null pointer argument");
  SMX_REQUIRE(rows >= 1 && rows < (1ll << 31) && vocab >= 1, "bad shape");
  SMX_REQUIRE((uintptr_t)out_ids % 8 == 0, "out_ids must be 8-byte aligned");
  SMX_LAUNCH(smx::argmax_kernel, dim3((unsigned)rows), dim3(1024), 0,
                     (hipStream_t)stream, (const uint16_t*)logits, vocab, out_ids);
  return (int)hipGetLastError();
}

extern "C" int smx_reshape_and_cache(void* stream, const void* key, const void* value,
                                     void* k_cache, void* v_cache, const int64_t* slot_mapping,
                                     int32_t num_tokens, int32_t n_kv, int32_t head_dim,
                                     int32_t num_blocks, int32_t block_size) {
  SMX_REQUIRE(key && value && k_cache && v_cache && slot_mapping, "null pointer argument");
  SMX_REQUIRE(num_tokens >= 1 && num_tokens <= 65535, "num_tokens must be in [1, 65535]");
  SMX_REQUIRE(n_kv >= 1 && n_kv <= 65535 && head_dim >= 1 && head_dim <= 4096, "bad head shape");
  SMX_REQUIRE(num_blocks >= 1 && block_size >= 1, "num_blocks and block_size must be >= 1");
  SMX_REQUIRE((uintptr_t)slot_mapping % 8 == 0, "slot_mapping must be 8-byte aligned");
  SMX_LAUNCH(smx::reshape_and_cache_kernel, dim3(n_kv, num_tokens), dim3(64), 0,
                     (hipStream_t)stream, (const uint16_t*)key, (const uint16_t*)value,
                     (uint16_t*)k_cache, (uint16_t*)v_cache, slot_mapping, n_kv, head_dim,
                     (int64_t)num_blocks * block_size);
  return (int)hipGetLastError();
}

extern "C" int smx_decode_advance(void* stream, int64_t* next_ids, const uint64_t* argmax_keys,
                                  int32_t num_keys, const int64_t* forced_ids,
                                  const int32_t* forced_len, int64_t* ids, int64_t* positions,
                                  int32_t* seq_lens, int64_t* slot_mapping,
                                  const int32_t* block_table, int64_t* tokens_out, int32_t rows,
                                  int32_t max_blocks, int32_t block_size, int32_t max_len,
                                  const void* embed_table, void* embed_out, int64_t vocab,
                                  int64_t hidden) {
  SMX_REQUIRE(next_ids && ids && positions && seq_lens && slot_mapping && block_table,
              "null pointer argument");
  SMX_REQUIRE(rows >= 1 && rows <= 65535 && max_blocks >= 1 && block_size >= 1 && max_len >= 0,
              "bad sizes");
  SMX_REQUIRE((forced_ids == nullptr) == (forced_len == nullptr),
              "forced_ids and forced_len go together");
  SMX_REQUIRE(!forced_ids || max_len >= 1, "forced_ids needs max_len >= 1");
  SMX_REQUIRE(!argmax_keys || num_keys >= 1, "argmax_keys needs num_keys >= 1");
  SMX_REQUIRE((uintptr_t)argmax_keys % 8 == 0, "argmax_keys must be 8-byte aligned");
  SMX_REQUIRE((embed_table == nullptr) == (embed_out == nullptr),
              "embed_table and embed_out go together");
  SMX_REQUIRE(!embed_table || (vocab >= 1 && hidden >= 1 && (uintptr_t)embed_table % 2 == 0 &&
                               (uintptr_t)embed_out % 2 == 0),
              "embedding needs vocab, hidden >= 1 and 2-byte aligned tables");
  const int nt = argmax_keys || embed_table ? 1024 : 64;
  SMX_LAUNCH(smx::decode_advance_kernel, dim3(rows), dim3(nt), 0, (hipStream_t)stream,
             next_ids, argmax_keys, num_keys, forced_ids, forced_len, ids, positions, seq_lens,
             slot_mapping, block_table, tokens_out, max_blocks, block_size, max_len,
             (const uint16_t*)embed_table, (uint16_t*)embed_out, vocab, hidden, nt);
  return (int)hipGetLastError();
}
extern "C" int smx_compute_slot_mapping(void* stream, const int32_t* query_start_loc,
                                        int32_t num_reqs, const int64_t* positions,
                                        const int32_t* block_table, int64_t* slot_mapping,
                                        int32_t num_tokens, int32_t max_tokens,
                                        int32_t max_blocks, int32_t block_size) {
  SMX_REQUIRE(query_start_loc && positions && block_table && slot_mapping,
              "null pointer argument");
  SMX_REQUIRE(num_reqs >= 1, "num_reqs must be >= 1");
  SMX_REQUIRE(num_tokens >= 0 && max_tokens >= 1 && num_tokens <= max_tokens,
              "need 0 <= num_tokens <= max_tokens, max_tokens >= 1");
  SMX_REQUIRE(max_blocks >= 1 && block_size >= 1, "max_blocks and block_size must be >= 1");
  SMX_REQUIRE((uintptr_t)positions % 8 == 0 && (uintptr_t)slot_mapping % 8 == 0 &&
                  (uintptr_t)query_start_loc % 4 == 0 && (uintptr_t)block_table % 4 == 0,
              "misaligned pointer");
  SMX_LAUNCH(smx::slot_mapping_kernel, dim3((max_tokens + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, query_start_loc, num_reqs, positions, block_table,
                     slot_mapping, num_tokens, max_tokens, max_blocks, block_size);
  return (int)hipGetLastError();
}
