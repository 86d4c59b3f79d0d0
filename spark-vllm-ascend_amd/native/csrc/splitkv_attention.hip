// Split-KV flash-decode attention over a paged bf16 KV cache, and the
// log-sum-exp merge of its partials, for gfx950.
//
// Semantics follow AttentionStage (src/spark_vllm_ascend/kernels/
// attention.py:59-117) and merge_attention (kernels/vector.py:45-83): per
// (split, kv head) an online softmax over the split's tokens, with the
// probabilities rounded to bf16 before they multiply V while the running sum
// keeps the fp32 values; each partial is normalised by its own sum and
// reported with lse = max + log(sum).
//
// Work decomposition (decode is HBM-bound: 512 bytes of K+V per token and kv
// head against ~2k flops): one workgroup per (kv head, split, sequence) whose
// waves stream 32- or 64-token blocks with all loads of a block in flight at
// once (details at splitkv_decode_kernel), then a separate merge kernel.
// Splits are either cut from the block table's capacity (one sequence: the
// first page lookups need no length) or taken from a per-step plan that cuts
// the batch's live tokens into equal per-sequence splits
// (splitkv_plan_kernel).  The merge is a second launch rather than a "last
// workgroup merges" epilogue: on this multi-XCD part the device-scope fence
// that epilogue needs writes back and invalidates each XCD's L2, which cost
// more than a launch.
#include <math.h>

#include <mutex>

#include "smx_common.h"
#include "smx_launch.h"

namespace smx {
namespace {

constexpr int HD = 128;
constexpr int G = 4;       // q heads per kv head
constexpr int TILE = 32;   // tokens per wave iteration

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));


// One workgroup of WAVES waves per (kv head, split, sequence).  Without a
// plan, split s covers [s*T, s*T + T) of the block table's capacity C
// (T = 32-aligned ceil(C / num_splits)), clipped to the sequence length; with
// a plan, workgroup y takes the token range of plan record y.  The WAVES waves
// take contiguous 32-aligned chunks of the split and walk them in BLK-token
// blocks, every K and V load of a block issued before any arithmetic; QK^T
// and PV run on v_mfma_f32_16x16x32_bf16 (operand layouts at load_block).
//
// Plan records (PLAN_WORDS uint32 words each, written by
// splitkv_plan_kernel): word 0 the sequence (-1: unused record), 1 / 2 the
// first / end token, 3 the split index within the sequence (bit 31 set when
// the plan was given positions and slots: only such a record can drive the
// fused q/k-norm + RoPE + KV write, which poisons its output with NaN and
// writes nothing to the cache otherwise), 4 the sequence length, 5-6 the
// position and 7-8 the slot (int64, little-endian), and words
// PLAN_PAGE0..63 the block-table entries from the first token's page on.
constexpr int PLAN_WORDS = 64;
constexpr int PLAN_PAGE0 = 9;
constexpr int PLAN_ALIGN = 128;  // split lengths are multiples of this (4 waves x 32 tokens)
constexpr uint32_t PLAN_HAS_POSITIONS = 0x80000000u;  // word 3 flag

struct SplitKVArgs {
  const uint16_t* q;  // [num_seqs, n_q, HD] (plain) or the raw QKV row (FUSEQ)
  const uint16_t* kc;
  uint16_t* vc_w;     // v cache (written by FUSEQ)
  uint16_t* kc_w;     // k cache (written by FUSEQ)
  const uint16_t* vc;
  const int32_t* block_table;
  const int32_t* seq_lens;
  float* part_o;
  float* part_lse;
  // FUSEQ only
  const uint16_t* q_gamma;
  const uint16_t* k_gamma;
  const uint16_t* cos_sin;
  const int64_t* positions;
  const int64_t* slot_mapping;
  int max_position;
  float eps;
  int num_splits, max_blocks, num_blocks, bs_log2, n_q, n_kv;
  float scale_log2;
};

// RMSNorm (gamma) + neox RoPE of one 128-wide head held by a wave as
// (a, b) = dims (lane, lane + 64) with gamma (ga, gb) at the same dims;
// returns the rotated pair as bf16 bits.
__device__ __forceinline__ void norm_rope_head(float a, float b, float ga, float gb, float c,
                                               float sn, float eps, uint16_t* u_out,
                                               uint16_t* v_out) {
  const float ss = wave_sum(a * a + b * b);
  const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
  const float an = round_bf16(a * inv * ga);
  const float bn = round_bf16(b * inv * gb);
  *u_out = f32_to_bf16(an * c - bn * sn);
  *v_out = f32_to_bf16(bn * c + an * sn);
}

// The arguments the first loads depend on are passed ahead of the rest as
// scalars and pointers (14 dwords): the library is built with kernel-argument
// preloading, which places leading non-aggregate arguments in SGPRs, so the
// first loads issue without a kernarg fetch.  pa_ / pb_ are the positions
// and slots (FUSEQ: the per-sequence gather reads them at entry) or the K and
// V caches (plain: read as soon as the first pages are known).
// lens_ is seq_lens, or with PLAN the plan records.
// With a plan, at least two waves per SIMD (left to itself the compiler
// gives the 4-wave 64-token variant 277 registers, one workgroup per CU);
// without, the compiler's choice (the one-sequence step measured 1.7% slower
// with the bound, which moves the MFMA accumulators out of AGPRs).
template <int WAVES, int BLK, bool FUSEQ, bool PLAN, bool RECFAST = false>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(PLAN ? 2 : 1)))
void splitkv_decode_kernel(
    const int32_t* block_table_, const void* lens_, const void* pa_, const void* pb_,
    const uint16_t* q_, int num_splits_, int max_blocks_, int bs_log2_, int n_kv_,
    SplitKVArgs A) {
  A.block_table = block_table_;
  A.seq_lens = (const int32_t*)lens_;
  if constexpr (FUSEQ) {
    A.positions = (const int64_t*)pa_;
    A.slot_mapping = (const int64_t*)pb_;
  } else {
    A.kc = (const uint16_t*)pa_;
    A.vc = (const uint16_t*)pb_;
  }
  A.q = q_;
  A.num_splits = num_splits_;
  A.max_blocks = max_blocks_;
  A.bs_log2 = bs_log2_;
  A.n_kv = n_kv_;
  A.n_q = 4 * n_kv_;  // GQA 4:1 (validated on the host)
  static_assert(BLK == 32 || BLK == 64, "blocks of 32 or 64 tokens");
  const uint16_t* __restrict__ kc = A.kc;
  const uint16_t* __restrict__ vc = A.vc;
  const int32_t* __restrict__ block_table = A.block_table;
  float* __restrict__ part_o = A.part_o;
  float* __restrict__ part_lse = A.part_lse;
  const int num_splits = A.num_splits, max_blocks = A.max_blocks, num_blocks = A.num_blocks;
  const int bs_log2 = A.bs_log2, n_q = A.n_q, n_kv = A.n_kv;
  const float scale_log2 = A.scale_log2;
  constexpr int NT = 64 * WAVES;
  __shared__ __attribute__((aligned(16))) uint32_t q_lds[G * HD / 2];  // 4 heads, bf16 pairs
  __shared__ __attribute__((aligned(16))) uint32_t p2[WAVES][2 * BLK];  // P: bf16 [head][token]
  __shared__ __attribute__((aligned(16))) float o_w[WAVES][G * HD];
  __shared__ float m_w[WAVES][G], l_w[WAVES][G];
  __shared__ int bad_w[WAVES];

  // Dispatch order is kv head fastest, then split (or plan record), then
  // sequence: the workgroups of one kv head share an XCD (workgroups go to the 8 XCDs
  // round-robin) and the 8 heads of the same tokens -- one 2 KB K row and
  // one V row per token -- are read together.  Measured: 2% off one
  // sequence's decode step against split-fastest; split-slowest made an
  // 8-sequence step 15% slower.  RECFAST (plans of 8k records): records
  // fastest, so the 8 heads of a record share one XCD instead (the launcher
  // says why).
  const int kvh = RECFAST ? blockIdx.y : blockIdx.x;
  const int rec = RECFAST ? blockIdx.x : blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cap = max_blocks << bs_log2;
  // The wave-uniform values this workgroup starts from come in ONE vector
  // load, one address per lane, read back with v_readlane: scalar loads would
  // each cost a full lgkmcnt(0) wait (their results return out of order), and
  // the compiler issues them one by one next to their uses.
  //  capacity splits: lane 0 the length, 3-4 the position, 5-6 the slot,
  //    lanes 8..63 the pages of the wave's chunk from its first one on;
  //  plan: the record (layout above).
  // With capacity splits the bounds follow from the block table's capacity,
  // not from the length, so all of it is one round trip; a plan record holds
  // the bounds and the first pages itself.
  constexpr int PB = PLAN ? PLAN_PAGE0 : 8;  // lane of the first gathered page
  constexpr int LEN_LANE = PLAN ? 4 : 0, POS_LANE = PLAN ? 5 : 3, SLOT_LANE = PLAN ? 7 : 5;
  uint32_t gv;
  int seq, split, s0, s_end, wlen, w0, pg0;
  bool pos_ok = true;  // FUSEQ: a position and a slot come with the split
  if constexpr (PLAN) {
    gv = reinterpret_cast<const uint32_t*>(lens_)[(int64_t)rec * PLAN_WORDS + lane];
    seq = __builtin_amdgcn_readlane((int)gv, 0);
    if (seq < 0) return;  // an unused record: the plan cleared the unused partials
    s0 = __builtin_amdgcn_readlane((int)gv, 1);
    s_end = __builtin_amdgcn_readlane((int)gv, 2);
    const uint32_t w3 = (uint32_t)__builtin_amdgcn_readlane((int)gv, 3);
    split = (int)(w3 & ~PLAN_HAS_POSITIONS);
    pos_ok = (w3 & PLAN_HAS_POSITIONS) != 0;
    wlen = ((s_end - s0 + WAVES - 1) / WAVES + TILE - 1) / TILE * TILE;
    w0 = min(s0 + wave * wlen, s_end);
    pg0 = s0 >> bs_log2;
  } else {
    split = blockIdx.y;
    seq = blockIdx.z;
    const int tps = ((cap + num_splits - 1) / num_splits + TILE - 1) / TILE * TILE;
    wlen = ((tps + WAVES - 1) / WAVES + TILE - 1) / TILE * TILE;
    s0 = split * tps;
    s_end = s0 + tps;
    w0 = min(s0 + wave * wlen, cap);
    pg0 = w0 < cap ? (w0 >> bs_log2) : 0;
    const uint32_t* src = reinterpret_cast<const uint32_t*>(A.seq_lens + seq);
    if constexpr (FUSEQ) {
      if (lane == 3 || lane == 4)
        src = reinterpret_cast<const uint32_t*>(A.positions + seq) + (lane - 3);
      if (lane == 5 || lane == 6)
        src = reinterpret_cast<const uint32_t*>(A.slot_mapping + seq) + (lane - 5);
    }
    if (lane >= 8)
      src = reinterpret_cast<const uint32_t*>(block_table + (int64_t)seq * max_blocks +
                                              min(pg0 + lane - 8, max_blocks - 1));
    gv = *src;
  }
  const int32_t* bt = block_table + (int64_t)seq * max_blocks;
  // FUSEQ: this workgroup's q heads and the new token's k/v from the raw QKV
  // row; with capacity splits they are issued in the same round trip (their
  // addresses need nothing loaded), with a plan right after the record.
  constexpr int HPW = (G + WAVES - 1) / WAVES;  // q heads per wave (FUSEQ)
  float qa[HPW], qb[HPW], qga = 0.f, qgb = 0.f, c = 0.f, sn = 0.f;
  float ka = 0.f, kb = 0.f, kga = 0.f, kgb = 0.f;
  uint16_t va = 0, vb = 0;
  const int nh = n_q + 2 * n_kv;
  const uint16_t* row = A.q + (int64_t)seq * nh * HD;
  if constexpr (FUSEQ) {
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int h = min(wave + i * WAVES, G - 1);
      qa[i] = bf16_bits_to_f32(row[(kvh * G + h) * HD + lane]);
      qb[i] = bf16_bits_to_f32(row[(kvh * G + h) * HD + 64 + lane]);
    }
    // the new token's k/v inputs (used by the owner's wave G % WAVES only)
    ka = bf16_bits_to_f32(row[(n_q + kvh) * HD + lane]);
    kb = bf16_bits_to_f32(row[(n_q + kvh) * HD + 64 + lane]);
    va = row[(n_q + n_kv + kvh) * HD + lane];
    vb = row[(n_q + n_kv + kvh) * HD + 64 + lane];
    qga = bf16_bits_to_f32(A.q_gamma[lane]);
    qgb = bf16_bits_to_f32(A.q_gamma[lane + 64]);
    kga = bf16_bits_to_f32(A.k_gamma[lane]);
    kgb = bf16_bits_to_f32(A.k_gamma[lane + 64]);
  }
  // Keep the scheduler from sinking those loads below the first use of the
  // gathered values (which waits for the gather): an empty asm that clobbers
  // memory orders the loads before it and emits no wait.
  __asm__ volatile("" ::: "memory");
  auto lane_u32 = [&](int l) -> uint32_t {
    return (uint32_t)__builtin_amdgcn_readlane((int)gv, l);
  };
  // page of token t >= the first gathered page: from the gather while it
  // covers t, else a block-table load
  auto page_of = [&](int t) -> int {
    const int li = (t >> bs_log2) - pg0 + PB;
    return li < 64 ? (int)lane_u32(li) : bt[min(t >> bs_log2, max_blocks - 1)];
  };
  // the first two pages: with capacity splits always gathered (lanes PB and
  // PB or PB + 1: no branch), with a plan maybe past the record
  const int bt0 = PLAN ? page_of(w0) : (int)lane_u32(PB);
  const int bt1 = PLAN ? page_of(w0 + 32) : (int)lane_u32(PB + (((w0 + 32) >> bs_log2) - pg0));
  const int L = min((int)lane_u32(LEN_LANE), cap);
  int64_t pos = 0;
  if constexpr (FUSEQ)
    pos = (int64_t)(((uint64_t)lane_u32(POS_LANE + 1) << 32) | lane_u32(POS_LANE));
  const int s1 = min(L, s_end);
  float* po = part_o + (((int64_t)seq * num_splits + split) * n_q + kvh * G) * HD;
  float* pl = part_lse + ((int64_t)seq * num_splits + split) * n_q + kvh * G;
  // An empty split (no token below the length) leaves (0, -inf).  Its exit
  // comes only now, after the gathered values arrived: the loads above are
  // already in flight, so the branch costs no round trip.
  if (s0 >= s1) {  // uniform over the workgroup
    for (int i = tid; i < G * HD; i += NT) st_agent(po + i, 0.f);
    if (tid < G) st_agent(pl + tid, -INFINITY);
    stores_done();
    return;
  }
  const int w1 = min(s1, w0 + wlen);

  const int bs = 1 << bs_log2;
  const int64_t tok_stride = (int64_t)n_kv * HD;
  const int64_t page_stride = tok_stride << bs_log2;

  // Lane roles of v_mfma_f32_16x16x32_bf16: lane l = 16 g + n holds row n of
  // A and column n of B at k = 8 g .. 8 g + 7, and rows 4 g .. 4 g + 3 of
  // column n of C.
  const int n = lane & 15, g = lane >> 4;

  // A block-table entry outside [0, num_blocks) is never dereferenced: the
  // page is replaced by page 0 and the partial is poisoned with NaN below.
  // A wave without tokens still issues its first block's loads, all from the
  // first row of page 0 (cached after the first touch, results unused):
  // loads under a branch would make the compiler wait for every outstanding
  // load before the q prologue.
  const bool has_work = w0 < w1;
  bool bad_page = false;
  auto half_base = [&](int t, int pg) -> int64_t {  // first token of a 32-token half
    if ((unsigned)pg >= (unsigned)num_blocks) {
      bad_page = bad_page || has_work;
      pg = 0;
    }
    if (!has_work) pg = t = 0;
    return (int64_t)pg * page_stride + (int64_t)(t & (bs - 1)) * tok_stride + kvh * HD;
  };
  // Every K and V load of one block, in the MFMA operand layouts; tokens past
  // the chunk end are loaded from the block's first token (always valid)
  // instead of branching, and their scores are masked to -inf.
  //  K (QK A operand, per 16-token tile tt and 32-dim step ks): token
  //    16 tt + n, dims 32 ks + 8 g .. + 8 -- 16 tokens x 64 bytes per load.
  //  V (per 32-token step sb, transposed in registers into the PV B
  //    operands): tokens 32 sb + 8 g + j (j < 8), dims 8 n .. 8 n + 7 -- four
  //    whole 256-byte rows per load.
  constexpr int NT16 = BLK / 16, NS32 = BLK / 32;
  u32x4 kr[NT16][4], vr[NS32][8];
  auto load_block = [&](int t0) {
    const int64_t b0 = half_base(t0, t0 == w0 ? bt0 : page_of(t0));
    const int64_t b1 = BLK == 64 && t0 + 32 < w1
                           ? half_base(t0 + 32, t0 == w0 ? bt1 : page_of(t0 + 32))
                           : b0;
    auto tok_off = [&](int t) -> int64_t {
      const int te = t0 + t < w1 ? t : 0;
      return (te < 32 ? b0 : b1) + (int64_t)(te & 31) * tok_stride;
    };
#pragma unroll
    for (int tt = 0; tt < NT16; ++tt) {
      const u32x4* kp = reinterpret_cast<const u32x4*>(kc + tok_off(16 * tt + n));
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) kr[tt][ks] = kp[4 * ks + g];
    }
#pragma unroll
    for (int sb = 0; sb < NS32; ++sb)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        vr[sb][j] = reinterpret_cast<const u32x4*>(vc + tok_off(32 * sb + 8 * g + j))[n];
  };
  // The rotary row (its address needs the position) and the first K/V block
  // (its pages) follow in the second round trip; the q/k norm + RoPE + KV
  // write run while the K/V block is in flight.
  __shared__ __attribute__((aligned(16))) uint32_t kv_new[2][HD / 2];
  bool owner = false;
  int64_t slot = -1;
  u32x4 qv = u32x4{0u, 0u, 0u, 0u};
  if constexpr (FUSEQ) {
    owner = pos_ok && pos >= s0 && pos < s1;
    const int64_t pc = pos < 0 ? 0 : (pos >= A.max_position ? A.max_position - 1 : pos);
    c = bf16_bits_to_f32(A.cos_sin[pc * HD + lane]);
    sn = bf16_bits_to_f32(A.cos_sin[pc * HD + 64 + lane]);
    slot = (int64_t)(((uint64_t)lane_u32(SLOT_LANE + 1) << 32) | lane_u32(SLOT_LANE));
  } else {
    qv = reinterpret_cast<const u32x4*>(A.q + ((int64_t)seq * n_q + kvh * G) * HD)[lane];
  }
  load_block(w0);

  if constexpr (FUSEQ) {
    uint16_t* qh = reinterpret_cast<uint16_t*>(q_lds);
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
      const int h = wave + i * WAVES;
      if (h < G)
        norm_rope_head(qa[i], qb[i], qga, qgb, c, sn, A.eps, &qh[h * HD + lane],
                       &qh[h * HD + 64 + lane]);
    }
    if (owner && wave == (G % WAVES)) {
      uint16_t* kn = reinterpret_cast<uint16_t*>(kv_new[0]);
      uint16_t* vn = reinterpret_cast<uint16_t*>(kv_new[1]);
      uint16_t ku, kv2;
      norm_rope_head(ka, kb, kga, kgb, c, sn, A.eps, &ku, &kv2);
      kn[lane] = ku;
      kn[lane + 64] = kv2;
      vn[lane] = va;
      vn[lane + 64] = vb;
      if (slot >= 0 && slot < ((int64_t)num_blocks << bs_log2)) {
        uint16_t* kd = A.kc_w + (slot * n_kv + kvh) * HD;
        uint16_t* vd = A.vc_w + (slot * n_kv + kvh) * HD;
        st_agent(kd + lane, ku);
        st_agent(kd + lane + 64, kv2);
        st_agent(vd + lane, va);
        st_agent(vd + lane + 64, vb);
      }
    }
  } else {
    if (tid < G * HD / 8) reinterpret_cast<u32x4*>(q_lds)[tid] = qv;
  }

  __syncthreads();
  // q as the QK B operand: column n = head n < G at the lane's dims (columns
  // n >= G are zero; their scores are computed and never used).
  u32x4 qop[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const u32x4 v = reinterpret_cast<const u32x4*>(q_lds)[(n & (G - 1)) * 16 + 4 * ks + g];
    qop[ks] = n < G ? v : u32x4{0u, 0u, 0u, 0u};
  }

  float m_mine = -INFINITY;  // running max (log2 domain) of head n (lanes n < G)
  float l_lane = 0.f;        // running sum of head n over this lane's tokens
  // PV accumulators, one C tile per dim group T: lane l < 16 holds heads
  // 0..3 of dim 8 l + T (rows 4..15 of every tile are the zero heads).
  f32x4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  uint16_t* pw = reinterpret_cast<uint16_t*>(p2[wave]);  // P as bf16 [head G][BLK]

  for (int t0 = w0; t0 < w1; t0 += BLK) {
    if (t0 != w0) load_block(t0);

    if constexpr (FUSEQ) {
      // The new token's K/V come from LDS (its cache slot is written by this
      // same launch, which does not order the store before these loads).
      const int tp = (int)(pos - t0);
      if (owner && tp >= 0 && tp < BLK) {
        const u32x4* kn = reinterpret_cast<const u32x4*>(kv_new[0]);
        const u32x4* vn = reinterpret_cast<const u32x4*>(kv_new[1]);
#pragma unroll
        for (int tt = 0; tt < NT16; ++tt)
          if (16 * tt + n == tp) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) kr[tt][ks] = kn[4 * ks + g];
          }
#pragma unroll
        for (int sb = 0; sb < NS32; ++sb)
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (32 * sb + 8 * g + j == tp) vr[sb][j] = vn[n];
      }
    }
    // ---- scores S[token][head]: lane (n, g) gets tokens 16 tt + 4 g + i of head n
    float sc[NT16][4];
#pragma unroll
    for (int tt = 0; tt < NT16; ++tt) {
      f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[tt][ks]),
                                                    __builtin_bit_cast(bf16x8, qop[ks]), c, 0, 0,
                                                    0);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sc[tt][i] = (t0 + 16 * tt + 4 * g + i < w1) ? c[i] * scale_log2 : -INFINITY;
    }
    // ---- online softmax (log2 domain) of head n over the lanes n + 16 g
    float mx = sc[0][0];
#pragma unroll
    for (int tt = 0; tt < NT16; ++tt)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sc[tt][i]);
    mx = xor_max<32>(xor_max<16>(mx));
    const float mn = fmaxf(m_mine, mx);
    const float alpha = exp2f(m_mine - mn);
    m_mine = mn;
    float psum = 0.f;
#pragma unroll
    for (int tt = 0; tt < NT16; ++tt) {
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = exp2f(sc[tt][i] - mn);
        psum += pv[i];
      }
      if (n < G)
        *reinterpret_cast<u32x2*>(pw + n * BLK + 16 * tt + 4 * g) =
            u32x2{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3])};
    }
    l_lane = l_lane * alpha + psum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- O = O * alpha + P V (the first block starts from O = 0)
    if (t0 != w0) {
      float alpha_h[G];
#pragma unroll
      for (int h = 0; h < G; ++h)
        alpha_h[h] = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), h));
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int r = 0; r < G; ++r) acc[t][r] *= alpha_h[r];
    }
#pragma unroll
    for (int sb = 0; sb < NS32; ++sb) {
      // A = P: row n = head n < G, tokens 32 sb + 8 g .. + 8
      const u32x4 pr = *reinterpret_cast<const u32x4*>(pw + (n & (G - 1)) * BLK + 32 * sb + 8 * g);
      const u32x4 pa = n < G ? pr : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        // B = V^T for dim group t: element 2i / 2i + 1 = tokens 8 g + 2i / + 1 at dim 8 n + t
        const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
        uint32_t bw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) bw[i] = perm_b32(vr[sb][2 * i + 1][t >> 1], vr[sb][2 * i][t >> 1], sel);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, pa),
                                                         __builtin_bit_cast(bf16x8, bw), acc[t],
                                                         0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- per-wave state to LDS
  const float l_tot = xor_sum<32>(xor_sum<16>(l_lane));
  if (lane < 16) {
#pragma unroll
    for (int r = 0; r < G; ++r) {
      float* dst = &o_w[wave][r * HD + 8 * lane];
      *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
    }
  }
  if (lane == 0) bad_w[wave] = bad_page || (FUSEQ && !pos_ok) ? 1 : 0;
  if (lane < G) {
    l_w[wave][lane] = l_tot;
    m_w[wave][lane] = m_mine;  // lane h keeps head h
  }
  __syncthreads();

  // ---- combine the waves: G*HD outputs
  int bad = 0;
#pragma unroll
  for (int wv = 0; wv < WAVES; ++wv) bad |= bad_w[wv];
  for (int e = tid; e < G * HD; e += NT) {
    const int h = e / HD;
    float mt = -INFINITY;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) mt = fmaxf(mt, m_w[wv][h]);
    float lt = 0.f, ot = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) {
      const float a = l_w[wv][h] > 0.f ? exp2f(m_w[wv][h] - mt) : 0.f;
      lt += a * l_w[wv][h];
      ot += a * o_w[wv][e];
    }
    // lt == 0 only when the split has no token: the empty partial (0, -inf)
    st_agent(po + e, bad ? __builtin_nanf("") : (lt > 0.f ? ot / lt : 0.f));
    if ((e % HD) == 0)
      st_agent(pl + h, bad ? __builtin_nanf("")
                           : (lt > 0.f ? (mt + log2f(lt)) * 0.69314718055994530942f : -INFINITY));
  }
  stores_done();
}

// Max / sum over the 64 lanes of a wave (every lane gets the result).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<DPP_QUAD_XOR1>(v));
  v = fmaxf(v, dpp_f32<DPP_QUAD_XOR2>(v));
  v = fmaxf(v, dpp_f32<DPP_ROW_HALF_MIRROR>(v));
  v = fmaxf(v, dpp_f32<DPP_ROW_MIRROR>(v));
  v = xor_max<16>(v);
  v = xor_max<32>(v);
  return v;
}

// Log-sum-exp merge (merge_attention, src/spark_vllm_ascend/kernels/
// vector.py:61-78): w_s = exp(lse_s - max), out = sum_s w_s o_s / sum_s w_s.
// One workgroup of nw waves per (64 dims of a q head, sequence); wave v folds
// the splits v, v + nw, v + 2 nw, ... in chunks of MCH: lane j loads the lse
// of the chunk's split j (one vector load) and lane d the chunk's partials of
// its dim, the chunk max and weight sum are wave reductions, and lane d folds
// its partials with the weights broadcast from their lanes (v_readlane).
// Every load of a chunk is unconditional (indices past the wave's last split
// are clamped, with uniform scalar arithmetic, and carry no weight), so a
// chunk costs one round trip; with nw = ceil(num_splits / MCH) waves each
// wave has a single chunk.  The waves then meet in LDS: the same merge over
// their (max, weight sum, weighted partial).  Splits with lse = -inf carry no
// weight; a NaN lse or partial makes the output NaN; no weight at all gives 0.
constexpr int MCH = 16;        // splits per wave per round trip
constexpr int MERGE_WAVES = 16;

__global__ __launch_bounds__(64 * MERGE_WAVES) void lse_merge_kernel(
    const float* __restrict__ part_o, const float* __restrict__ part_lse,
    uint16_t* __restrict__ out, int num_splits, int n_q, int nw) {
  __shared__ float m_s[MERGE_WAVES], l_s[MERGE_WAVES], a_s[MERGE_WAVES][64];
  __shared__ int bad_s[MERGE_WAVES];
  // Workgroup b serves kv head b % n_kv (its 2 G head halves are b / n_kv):
  // workgroups go to the XCDs round-robin by linear id, and the attention
  // kernel's workgroups of kv head j (kv heads fastest) run on XCD j % 8, so
  // with n_kv = 8 a head's partials are read on the XCD whose L2 wrote them.
  // (n_q not a multiple of G: workgroup b serves head b / 2, half b % 2.)
  const int n_kv = n_q % G == 0 ? n_q / G : n_q;
  const int kvh = blockIdx.x % n_kv, j = blockIdx.x / n_kv;
  const int h = n_q % G == 0 ? kvh * G + (j >> 1) : (int)blockIdx.x >> 1;
  const int half = n_q % G == 0 ? (j & 1) : (int)blockIdx.x & 1;
  const int seq = blockIdx.y;
  const int lane = threadIdx.x & 63, d = half * 64 + lane;
  const int v = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)seq * num_splits * n_q + h;  // (seq, split 0, h)
  const int cnt = v < num_splits ? (num_splits - 1 - v) / nw + 1 : 0;  // this wave's splits
  const int64_t sstep = (int64_t)nw * n_q;                           // split v -> v + nw
  float m = -INFINITY, l = 0.f, acc = 0.f;
  bool poisoned = false;
  for (int i0 = 0; i0 < cnt; i0 += MCH) {
    const int last = min(cnt - 1 - i0, MCH - 1);  // last valid j of this chunk (uniform)
    const int64_t c0 = row + ((int64_t)v + (int64_t)i0 * nw) * n_q;  // split v + nw i0
    const float lraw = part_lse[c0 + (int64_t)min(lane, last) * sstep];
    float pv[MCH];
    const float* pp = part_o + c0 * HD + d;
    int64_t off = 0;  // element offset of split v + nw (i0 + min(j, last))
#pragma unroll
    for (int j = 0; j < MCH; ++j) {
      pv[j] = pp[off];
      off += j < last ? sstep * HD : 0;
    }
    // every load of the chunk is issued before the wait for its lse values
    // (nothing may be scheduled across this point)
    __builtin_amdgcn_sched_barrier(0);
    const float lv = lane <= last ? lraw : -INFINITY;
    poisoned |= __builtin_amdgcn_ballot_w64(lv != lv) != 0;
    // Branch-free (a branch would let the compiler sink the partial loads
    // behind the lse wait): with no weight so far both factors are 0.
    const float mc = fmaxf(m, wave_max(lv));
    const float wl = lv == -INFINITY ? 0.f : expf(lv - mc);
    const float a = m == -INFINITY ? 0.f : expf(m - mc);
    l = l * a + wave_sum(wl);
    acc *= a;
#pragma unroll
    for (int j = 0; j < MCH; ++j) {
      const float wj = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), j));
      acc = fmaf(wj, pv[j], acc);
    }
    m = mc;
  }
  if (nw > 1) {
    a_s[v][lane] = acc;
    if (lane == 0) {
      m_s[v] = m;
      l_s[v] = l;
      bad_s[v] = poisoned ? 1 : 0;
    }
    __syncthreads();
    if (v != 0) return;
    float mt = -INFINITY;
    for (int w = 0; w < nw; ++w) mt = fmaxf(mt, m_s[w]);
    l = 0.f;
    acc = 0.f;
    for (int w = 0; w < nw; ++w) {
      const float f = m_s[w] == -INFINITY ? 0.f : expf(m_s[w] - mt);
      l = fmaf(f, l_s[w], l);
      acc = fmaf(f, a_s[w][lane], acc);
      poisoned |= bad_s[w] != 0;
    }
  }
  const float r = poisoned || acc != acc ? __builtin_nanf("") : (l > 0.f ? acc / l : 0.f);
  st_agent(out + ((int64_t)seq * n_q + h) * HD + d, f32_to_bf16(r));
  stores_done();
}


// Per-sequence split plan for a batch of decode sequences (the device-side
// task list of execute_serial, src/spark_vllm_ascend/kernels/attention.py:
// 120-128, where parts = ceil(length / width) follows the live length): the
// batch's T = sum_r L_r live tokens are cut into splits of one length
//   chunk = PLAN_ALIGN * ceil(max(ceil(T / num_items),
//                                 ceil(max_r L_r / num_splits), 1) / PLAN_ALIGN)
// that never cross a sequence, so sequence r has n_r = ceil(L_r / chunk) <=
// num_splits splits and sum_r n_r <= num_items + num_seqs (the record count).
// Items are numbered sequence by sequence; record b describes item b, or is
// unused (sequence -1) past the last item.  Every workgroup reads all lengths
// (one per lane, num_seqs <= 64) and derives the same plan; workgroup b
// writes record b and clears partial slot b = (sequence, split) when no item
// writes it (partial 0, lse -inf), so the merge over num_splits slots sees
// empty splits there.  One launch serves every layer of a decode step.
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

__device__ __forceinline__ int wave_max_i32(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = max(v, __shfl_xor(v, o));
  return v;
}

__global__ __launch_bounds__(64) void splitkv_plan_kernel(
    const int32_t* __restrict__ seq_lens, const int64_t* __restrict__ positions,
    const int64_t* __restrict__ slot_mapping, const int32_t* __restrict__ block_table,
    uint32_t* __restrict__ plan, float* __restrict__ part_o, float* __restrict__ part_lse,
    int num_seqs, int num_items, int num_splits, int max_blocks, int bs_log2, int n_q) {
  const int lane = threadIdx.x;
  const int b = blockIdx.x;
  const int cap = max_blocks << bs_log2;
  const int L = lane < num_seqs ? min(max(seq_lens[lane], 0), cap) : 0;
  const int total = wave_sum_i32(L);  // <= num_seqs * cap < 2^31 (checked on the host)
  const int lmax = wave_max_i32(L);
  int chunk = max(max((total + num_items - 1) / num_items, (lmax + num_splits - 1) / num_splits), 1);
  chunk = (chunk + PLAN_ALIGN - 1) / PLAN_ALIGN * PLAN_ALIGN;
  const int n = (L + chunk - 1) / chunk;  // splits of this lane's sequence
  int incl = n;                           // inclusive prefix sum over the lanes
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  const int n_items = __shfl(incl, 63);
  if (b < num_items + num_seqs) {
    uint32_t w = lane == 0 ? 0xffffffffu : 0u;  // unused record
    if (b < n_items) {
      // the sequence holding item b: the first lane whose prefix passes b
      const int i = __ffsll((unsigned long long)__ballot(incl > b)) - 1;
      const int li = __shfl(L, i);
      const int j = b - (__shfl(incl, i) - __shfl(n, i));
      const int tb = j * chunk, te = min(tb + chunk, li);
      const int64_t p = positions ? positions[i] : 0;
      const int64_t sl = slot_mapping ? slot_mapping[i] : -1;
      const uint32_t flag = positions && slot_mapping ? PLAN_HAS_POSITIONS : 0u;
      const uint32_t head[PLAN_PAGE0] = {(uint32_t)i, (uint32_t)tb, (uint32_t)te, (uint32_t)j | flag,
                                         (uint32_t)li, (uint32_t)p, (uint32_t)(p >> 32),
                                         (uint32_t)sl, (uint32_t)(sl >> 32)};
      if (lane < PLAN_PAGE0) {
#pragma unroll
        for (int k = 0; k < PLAN_PAGE0; ++k)
          if (lane == k) w = head[k];
      } else {
        w = (uint32_t)block_table[(int64_t)i * max_blocks +
                                  min((tb >> bs_log2) + lane - PLAN_PAGE0, max_blocks - 1)];
      }
    }
    st_agent(plan + (int64_t)b * PLAN_WORDS + lane, w);
  }
  if (b < num_seqs * num_splits) {
    const int seq = b / num_splits;
    if (b - seq * num_splits >= __shfl(n, seq)) {
      u32x4* po = reinterpret_cast<u32x4*>(part_o + (int64_t)b * n_q * HD);
      for (int e = lane; e < n_q * HD / 4; e += 64) st_agent(po + e, u32x4{0u, 0u, 0u, 0u});
      for (int h = lane; h < n_q; h += 64) st_agent(part_lse + (int64_t)b * n_q + h, -INFINITY);
    }
  }
  stores_done();
}

}  // namespace
}  // namespace smx

#include "smx_abi_util.h"

namespace {
// plan: the plan records (num_records of them), or null for capacity splits.
template <bool FUSEQ>
int launch_splitkv(void* stream, smx::SplitKVArgs a, int32_t num_seqs, int32_t block_size,
                   float scale, const uint32_t* plan = nullptr, int num_records = 0) {
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  a.bs_log2 = bs_log2;
  a.scale_log2 = scale * 1.44269504088896340736f;
  // Blocks of 32 tokens (shorter per-wave dependency chains) while a split
  // fits 8 such waves, else 64-token blocks over 8 waves.
  const int64_t cap = (int64_t)a.max_blocks * block_size;
  const int64_t tps = ((cap + a.num_splits - 1) / a.num_splits + 31) / 32 * 32;
  int blk = tps <= 256 ? 32 : 64;
  int waves = blk == 64 ? 8 : tps <= 32 ? 1 : tps <= 64 ? 2 : tps <= 128 ? 4 : 8;
  // A plan's splits are long (the batch's tokens over a few hundred
  // workgroups): 2 waves of 32-token blocks per workgroup, each wave half a
  // split (8-sequence step: 2 waves 4.69-4.72 ms, 4 waves 4.72-4.74, 1 wave
  // 5.06; 64-token blocks take 246 VGPRs and measured 5.02).
  if (plan) {
    blk = 32;
    waves = 2;
  }
  const char* e = smx::tuning_env("SMX_ATTN_WAVES");  // "waves[,blk]" override for tuning sweeps
  if (e) {
    int w = 0, b = 0;
    const int n = sscanf(e, "%d,%d", &w, &b);
    if (n >= 1 && (w == 1 || w == 2 || w == 4 || w == 8)) waves = w;
    if (n == 2 && (b == 32 || b == 64)) blk = b;
  }
  // A plan of 8k records runs records fastest: workgroups go to the XCDs
  // round-robin by linear id (record + records * kv head), so all kv heads of
  // one record share an XCD and its requests cover whole token rows
  // (8-sequence step, 96 records: attention 88.6 against 90.8-91.4 µs per
  // layer, the step 4.597 against 4.675 ms).  Capacity splits keep kv heads
  // fastest: the merge reads a kv head's partials on that head's XCD.
  const bool recfast = plan && num_records % 8 == 0;
  const dim3 grid = plan ? (recfast ? dim3(num_records, a.n_kv, 1) : dim3(a.n_kv, num_records, 1))
                         : dim3(a.n_kv, a.num_splits, num_seqs);
#define SMX_ATTN_LAUNCH(W, B)                                                                   \
  do {                                                                                          \
    if (plan && recfast)                                                                        \
      SMX_LAUNCH((smx::splitkv_decode_kernel<W, B, FUSEQ, true, true>), grid,           \
                         dim3(64 * W), 0, (hipStream_t)stream, a.block_table, (const void*)plan,  \
                         FUSEQ ? (const void*)a.positions : (const void*)a.kc,                     \
                         FUSEQ ? (const void*)a.slot_mapping : (const void*)a.vc, a.q,             \
                         a.num_splits, a.max_blocks, a.bs_log2, a.n_kv, a);                        \
    else if (plan)                                                                              \
      SMX_LAUNCH((smx::splitkv_decode_kernel<W, B, FUSEQ, true>), grid, dim3(64 * W),   \
                         0, (hipStream_t)stream, a.block_table, (const void*)plan,                \
                         FUSEQ ? (const void*)a.positions : (const void*)a.kc,                     \
                         FUSEQ ? (const void*)a.slot_mapping : (const void*)a.vc, a.q,             \
                         a.num_splits, a.max_blocks, a.bs_log2, a.n_kv, a);                        \
    else                                                                                        \
      SMX_LAUNCH((smx::splitkv_decode_kernel<W, B, FUSEQ, false>), grid, dim3(64 * W),  \
                         0, (hipStream_t)stream, a.block_table, (const void*)a.seq_lens,          \
                         FUSEQ ? (const void*)a.positions : (const void*)a.kc,                     \
                         FUSEQ ? (const void*)a.slot_mapping : (const void*)a.vc, a.q,             \
                         a.num_splits, a.max_blocks, a.bs_log2, a.n_kv, a);                        \
  } while (0)
  if (blk == 32) {
    if (waves == 8) SMX_ATTN_LAUNCH(8, 32);
    else if (waves == 4) SMX_ATTN_LAUNCH(4, 32);
    else if (waves == 2) SMX_ATTN_LAUNCH(2, 32);
    else SMX_ATTN_LAUNCH(1, 32);
  } else {
    if (waves == 8) SMX_ATTN_LAUNCH(8, 64);
    else if (waves == 4) SMX_ATTN_LAUNCH(4, 64);
    else if (waves == 2) SMX_ATTN_LAUNCH(2, 64);
    else SMX_ATTN_LAUNCH(1, 64);
  }
#undef SMX_ATTN_LAUNCH
  return (int)hipGetLastError();
}

smx::SplitKVArgs splitkv_args(const void* q, const void* k_cache, const void* v_cache,
                              const int32_t* block_table, const int32_t* seq_lens,
                              float* partial_o, float* partial_lse, int32_t num_splits,
                              int32_t max_blocks, int32_t num_blocks, int32_t n_q,
                              int32_t n_kv) {
  smx::SplitKVArgs a{};
  a.q = (const uint16_t*)q;
  a.kc = (const uint16_t*)k_cache;
  a.vc = (const uint16_t*)v_cache;
  a.kc_w = (uint16_t*)k_cache;
  a.vc_w = (uint16_t*)v_cache;
  a.block_table = block_table;
  a.seq_lens = seq_lens;
  a.part_o = partial_o;
  a.part_lse = partial_lse;
  a.num_splits = num_splits;
  a.max_blocks = max_blocks;
  a.num_blocks = num_blocks;
  a.n_q = n_q;
  a.n_kv = n_kv;
  return a;
}

int launch_merge(void* stream, const float* partial_o, const float* partial_lse, void* out,
                 int32_t num_seqs, int32_t num_splits, int32_t n_q) {
  // one chunk per wave where possible (at most MERGE_WAVES waves)
  const int nw = std::min((num_splits + smx::MCH - 1) / smx::MCH, smx::MERGE_WAVES);
  SMX_LAUNCH(smx::lse_merge_kernel, dim3(2 * n_q, num_seqs), dim3(64 * nw), 0,
                     (hipStream_t)stream, partial_o, partial_lse, (uint16_t*)out, num_splits,
                     n_q, nw);
  return (int)hipGetLastError();
}
}  // namespace

#define SMX_SPLITKV_CHECKS()                                                                     \
  SMX_REQUIRE(q && k_cache && v_cache && block_table && seq_lens && partial_o && partial_lse,    \
              "null pointer argument");                                                          \
  SMX_REQUIRE(num_seqs >= 1 && num_seqs <= 65535, "num_seqs must be in [1, 65535]");             \
  SMX_REQUIRE(num_splits >= 1 && num_splits <= 4096, "num_splits must be in [1, 4096]");         \
  SMX_REQUIRE(max_blocks >= 1 && num_blocks >= 1, "max_blocks and num_blocks must be >= 1");     \
  SMX_REQUIRE(head_dim == 128, "head_dim must be 128");                                          \
  SMX_REQUIRE(n_kv >= 1 && n_q == 4 * n_kv && n_kv <= 65535, "need n_q == 4 * n_kv (GQA 4:1)"); \
  SMX_REQUIRE(block_size >= 32 && block_size <= 4096 && (block_size & (block_size - 1)) == 0,    \
              "block_size must be a power of two in [32, 4096]");                                \
  SMX_REQUIRE((int64_t)max_blocks * block_size <= INT32_MAX,                                     \
              "max_blocks * block_size (a sequence's capacity) must fit in int32");              \
  SMX_REQUIRE(scale > 0.f && isfinite(scale), "scale must be positive and finite");              \
  SMX_REQUIRE((uintptr_t)q % 16 == 0 && (uintptr_t)k_cache % 16 == 0 &&                          \
                  (uintptr_t)v_cache % 16 == 0 && (uintptr_t)block_table % 4 == 0 &&             \
                  (uintptr_t)seq_lens % 4 == 0 && (uintptr_t)partial_o % 4 == 0 &&               \
                  (uintptr_t)partial_lse % 4 == 0,                                               \
              "q, k_cache and v_cache must be 16-byte aligned; int/float arrays 4-byte aligned")

extern "C" int smx_splitkv_decode(void* stream, const void* q, const void* k_cache,
                                  const void* v_cache, const int32_t* block_table,
                                  const int32_t* seq_lens, float* partial_o, float* partial_lse,
                                  int32_t num_seqs, int32_t num_splits, int32_t max_blocks,
                                  int32_t num_blocks, int32_t block_size, int32_t n_q,
                                  int32_t n_kv, int32_t head_dim, float scale) {
  SMX_SPLITKV_CHECKS();
  return launch_splitkv<false>(stream,
                               splitkv_args(q, k_cache, v_cache, block_table, seq_lens,
                                            partial_o, partial_lse, num_splits, max_blocks,
                                            num_blocks, n_q, n_kv),
                               num_seqs, block_size, scale);
}

extern "C" int smx_splitkv_decode_merged(void* stream, const void* q, const void* k_cache,
                                         const void* v_cache, const int32_t* block_table,
                                         const int32_t* seq_lens, float* partial_o,
                                         float* partial_lse, void* out, int32_t num_seqs,
                                         int32_t num_splits, int32_t max_blocks,
                                         int32_t num_blocks, int32_t block_size, int32_t n_q,
                                         int32_t n_kv, int32_t head_dim, float scale) {
  SMX_SPLITKV_CHECKS();
  SMX_REQUIRE(out && (uintptr_t)out % 2 == 0, "out must be non-null and 2-byte aligned");
  const int rc = launch_splitkv<false>(stream,
                                       splitkv_args(q, k_cache, v_cache, block_table, seq_lens,
                                                    partial_o, partial_lse, num_splits,
                                                    max_blocks, num_blocks, n_q, n_kv),
                                       num_seqs, block_size, scale);
  if (rc) return rc;
  return launch_merge(stream, partial_o, partial_lse, out, num_seqs, num_splits, n_q);
}

// ---------------------------------------------------------------------------
// smx_splitkv_decode_merged_noalloc: the same two launches, with the split
// partials in a file-scope device array instead of caller buffers, for callers
// that cannot allocate.  Every GPU the library runs on holds its own copy of
// the array until the process ends.  In host code `scratch` names a host-side
// stand-in, not device memory: its device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only
// that address is handed to kernels.  All calls on one GPU share the array,
// so calls that overlap on one GPU (different streams, or graphs replayed
// concurrently) race.  Nothing needs clearing between calls: the decode
// kernel writes every (sequence, split) slot the merge reads, an empty split
// included.
// ---------------------------------------------------------------------------
namespace {
static __device__ __align__(256) unsigned char scratch[SMX_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch array (resolved on first use), or
// nullptr with *rc set to the HIP error.
void* scratch_for_current_device(int* rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = (int)e;
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = (int)hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
      return nullptr;
    }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

// Bytes of scratch a call uses: the partials, then (256-byte aligned) the lse.
int64_t noalloc_bytes(int32_t num_seqs, int32_t num_splits, int32_t n_q, int32_t head_dim) {
  if (num_seqs < 1 || num_splits < 1 || n_q < 1 || head_dim < 1) return -1;
  const int64_t slots = (int64_t)num_seqs * num_splits * n_q;
  const int64_t o_bytes = (slots * head_dim * 4 + 255) / 256 * 256;
  return o_bytes + slots * 4;
}
}  // namespace

extern "C" int smx_splitkv_decode_merged_noalloc(void* stream, const void* q, const void* k_cache,
                                                 const void* v_cache, const int32_t* block_table,
                                                 const int32_t* seq_lens, void* out,
                                                 int32_t num_seqs, int32_t num_splits,
                                                 int32_t max_blocks, int32_t num_blocks,
                                                 int32_t block_size, int32_t n_q, int32_t n_kv,
                                                 int32_t head_dim, float scale) {
  // the partial pointers are checked below, once the scratch address is known
  const float* partial_o = reinterpret_cast<const float*>(16);
  const float* partial_lse = partial_o;
  SMX_SPLITKV_CHECKS();
  SMX_REQUIRE(out && (uintptr_t)out % 2 == 0, "out must be non-null and 2-byte aligned");
  const int64_t need = noalloc_bytes(num_seqs, num_splits, n_q, head_dim);
  SMX_REQUIRE(need > 0 && need <= (int64_t)SMX_NOALLOC_SCRATCH_BYTES,
              "num_seqs * num_splits * n_q * (4 * head_dim + 4) bytes (with the lse block "
              "256-byte aligned) exceed SMX_NOALLOC_SCRATCH_BYTES; use "
              "smx_splitkv_decode_merged with caller buffers");
  int rc = 0;
  unsigned char* base = static_cast<unsigned char*>(scratch_for_current_device(&rc));
  if (!base) return rc;
  const int64_t o_bytes = need - (int64_t)num_seqs * num_splits * n_q * 4;
  float* po = reinterpret_cast<float*>(base);
  float* pl = reinterpret_cast<float*>(base + o_bytes);
  rc = launch_splitkv<false>(stream,
                             splitkv_args(q, k_cache, v_cache, block_table, seq_lens, po, pl,
                                          num_splits, max_blocks, num_blocks, n_q, n_kv),
                             num_seqs, block_size, scale);
  if (rc) return rc;
  return launch_merge(stream, po, pl, out, num_seqs, num_splits, n_q);
}

extern "C" int smx_qknorm_rope_splitkv_decode_merged(
    void* stream, const void* qkv, const void* q_gamma, const void* k_gamma,
    const void* cos_sin, const int64_t* positions, const int64_t* slot_mapping, void* k_cache,
    void* v_cache, const int32_t* block_table, const int32_t* seq_lens, float* partial_o,
    float* partial_lse, void* out, int32_t num_seqs, int32_t num_splits, int32_t max_blocks,
    int32_t num_blocks, int32_t block_size, int32_t n_q, int32_t n_kv, int32_t head_dim,
    int32_t max_position, float eps, float scale) {
  const void* q = qkv;
  SMX_SPLITKV_CHECKS();
  SMX_REQUIRE(q_gamma && k_gamma && cos_sin && positions && slot_mapping && out,
              "null pointer argument");
  SMX_REQUIRE(max_position >= 1, "max_position must be >= 1");
  SMX_REQUIRE(eps >= 0.f && isfinite(eps), "eps must be finite and >= 0");
  SMX_REQUIRE((uintptr_t)positions % 8 == 0 && (uintptr_t)slot_mapping % 8 == 0 &&
                  (uintptr_t)out % 2 == 0 && (uintptr_t)q_gamma % 2 == 0 &&
                  (uintptr_t)k_gamma % 2 == 0 && (uintptr_t)cos_sin % 2 == 0,
              "misaligned pointer");
  smx::SplitKVArgs a = splitkv_args(qkv, k_cache, v_cache, block_table, seq_lens, partial_o,
                                    partial_lse, num_splits, max_blocks, num_blocks, n_q, n_kv);
  a.q_gamma = (const uint16_t*)q_gamma;
  a.k_gamma = (const uint16_t*)k_gamma;
  a.cos_sin = (const uint16_t*)cos_sin;
  a.positions = positions;
  a.slot_mapping = slot_mapping;
  a.max_position = max_position;
  a.eps = eps;
  const int rc = launch_splitkv<true>(stream, a, num_seqs, block_size, scale);
  if (rc) return rc;
  return launch_merge(stream, partial_o, partial_lse, out, num_seqs, num_splits, n_q);
}

extern "C" int smx_lse_merge(void* stream, const float* partial_o, const float* partial_lse,
                             void* out, int32_t num_seqs, int32_t num_splits, int32_t n_q,
                             int32_t head_dim) {
  SMX_REQUIRE(partial_o && partial_lse && out, "null pointer argument");
  SMX_REQUIRE(num_seqs >= 1 && num_seqs <= 65535, "num_seqs must be in [1, 65535]");
  SMX_REQUIRE(num_splits >= 1 && num_splits <= 4096, "num_splits must be in [1, 4096]");
  SMX_REQUIRE(head_dim == 128 && n_q >= 1 && n_q <= 65535, "head_dim must be 128");
  SMX_REQUIRE((uintptr_t)out % 2 == 0 && (uintptr_t)partial_o % 4 == 0 &&
                  (uintptr_t)partial_lse % 4 == 0,
              "misaligned pointer");
  return launch_merge(stream, partial_o, partial_lse, out, num_seqs, num_splits, n_q);
}

#define SMX_PLAN_CHECKS()                                                                        \
  SMX_REQUIRE(plan, "null plan");                                                                \
  SMX_REQUIRE(num_seqs <= 64, "a plan covers at most 64 sequences");                             \
  SMX_REQUIRE(num_items >= 1 && num_items + num_seqs <= 65535,                                   \
              "num_items must be >= 1 with num_items + num_seqs <= 65535");                      \
  SMX_REQUIRE((uintptr_t)plan % 4 == 0, "plan must be 4-byte aligned")

extern "C" int smx_splitkv_plan(void* stream, const int32_t* seq_lens, const int64_t* positions,
                                const int64_t* slot_mapping, const int32_t* block_table,
                                uint32_t* plan, float* partial_o, float* partial_lse,
                                int32_t num_seqs, int32_t num_items, int32_t num_splits,
                                int32_t max_blocks, int32_t block_size, int32_t n_q,
                                int32_t head_dim) {
  SMX_REQUIRE(seq_lens && block_table && partial_o && partial_lse, "null pointer argument");
  SMX_REQUIRE(num_seqs >= 1, "num_seqs must be >= 1");
  SMX_PLAN_CHECKS();
  SMX_REQUIRE(num_splits >= 1 && num_splits <= 4096, "num_splits must be in [1, 4096]");
  SMX_REQUIRE(max_blocks >= 1, "max_blocks must be >= 1");
  SMX_REQUIRE(block_size >= 32 && block_size <= 4096 && (block_size & (block_size - 1)) == 0,
              "block_size must be a power of two in [32, 4096]");
  SMX_REQUIRE((int64_t)num_seqs * max_blocks * block_size <= INT32_MAX,
              "num_seqs * max_blocks * block_size must fit in int32");
  SMX_REQUIRE(head_dim == 128 && n_q >= 1 && n_q <= 65535, "head_dim must be 128");
  SMX_REQUIRE((uintptr_t)seq_lens % 4 == 0 && (uintptr_t)block_table % 4 == 0 &&
                  (uintptr_t)positions % 8 == 0 && (uintptr_t)slot_mapping % 8 == 0 &&
                  (uintptr_t)partial_o % 16 == 0 && (uintptr_t)partial_lse % 4 == 0,
              "misaligned pointer (partial_o needs 16 bytes)");
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  const int64_t grid = std::max<int64_t>(num_items + num_seqs, (int64_t)num_seqs * num_splits);
  SMX_LAUNCH(smx::splitkv_plan_kernel, dim3((unsigned)grid), dim3(64), 0,
                     (hipStream_t)stream, seq_lens, positions, slot_mapping, block_table, plan,
                     partial_o, partial_lse, num_seqs, num_items, num_splits, max_blocks, bs_log2,
                     n_q);
  return (int)hipGetLastError();
}

extern "C" int smx_splitkv_decode_planned_merged(
    void* stream, const void* q, const void* k_cache, const void* v_cache,
    const int32_t* block_table, const uint32_t* plan, float* partial_o, float* partial_lse,
    void* out, int32_t num_seqs, int32_t num_items, int32_t num_splits, int32_t max_blocks,
    int32_t num_blocks, int32_t block_size, int32_t n_q, int32_t n_kv, int32_t head_dim,
    float scale) {
  const void* seq_lens = plan;  // the plan's records carry the lengths
  SMX_SPLITKV_CHECKS();
  SMX_PLAN_CHECKS();
  SMX_REQUIRE(out && (uintptr_t)out % 2 == 0, "out must be non-null and 2-byte aligned");
  const int rc = launch_splitkv<false>(
      stream,
      splitkv_args(q, k_cache, v_cache, block_table, nullptr, partial_o, partial_lse, num_splits,
                   max_blocks, num_blocks, n_q, n_kv),
      num_seqs, block_size, scale, plan, num_items + num_seqs);
  if (rc) return rc;
  return launch_merge(stream, partial_o, partial_lse, out, num_seqs, num_splits, n_q);
}

extern "C" int smx_qknorm_rope_splitkv_decode_planned_merged(
    void* stream, const void* qkv, const void* q_gamma, const void* k_gamma,
    const void* cos_sin, void* k_cache, void* v_cache, const int32_t* block_table,
    const uint32_t* plan, float* partial_o, float* partial_lse, void* out, int32_t num_seqs,
    int32_t num_items, int32_t num_splits, int32_t max_blocks, int32_t num_blocks,
    int32_t block_size, int32_t n_q, int32_t n_kv, int32_t head_dim, int32_t max_position,
    float eps, float scale) {
  const void* q = qkv;
  const void* seq_lens = plan;  // the plan's records carry lengths, positions and slots
  SMX_SPLITKV_CHECKS();
  SMX_PLAN_CHECKS();
  SMX_REQUIRE(q_gamma && k_gamma && cos_sin && out, "null pointer argument");
  SMX_REQUIRE(max_position >= 1, "max_position must be >= 1");
  SMX_REQUIRE(eps >= 0.f && isfinite(eps), "eps must be finite and >= 0");
  SMX_REQUIRE((uintptr_t)out % 2 == 0 && (uintptr_t)q_gamma % 2 == 0 &&
                  (uintptr_t)k_gamma % 2 == 0 && (uintptr_t)cos_sin % 2 == 0,
              "misaligned pointer");
  smx::SplitKVArgs a = splitkv_args(qkv, k_cache, v_cache, block_table, nullptr, partial_o,
                                    partial_lse, num_splits, max_blocks, num_blocks, n_q, n_kv);
  a.q_gamma = (const uint16_t*)q_gamma;
  a.k_gamma = (const uint16_t*)k_gamma;
  a.cos_sin = (const uint16_t*)cos_sin;
  a.max_position = max_position;
  a.eps = eps;
  const int rc = launch_splitkv<true>(stream, a, num_seqs, block_size, scale, plan,
                                      num_items + num_seqs);
  if (rc) return rc;
  return launch_merge(stream, partial_o, partial_lse, out, num_seqs, num_splits, n_q);
}
