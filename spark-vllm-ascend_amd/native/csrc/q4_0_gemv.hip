// Q4_0 (GGUF type 2) dequantisation and dequant-fused GEMV for gfx950.
//
// A Q4_0 row of k weights is k/32 blocks of 18 bytes: an fp16 scale d and 16
// bytes qs holding element j (j < 16) in the low nibble of qs[j] and element
// 16 + j in its high nibble; value = d * (nibble - 8).  This is the block
// decode of src/spark_vllm_ascend/integration/weights.py:34-40.
//
// GEMV design (M = 1 is HBM-bound: 18 bytes per 32 weights, ~3.5 flop/B):
//  * The weights are streamed in their GGUF layout.  A lane owns a block
//    PAIR (36 bytes, 4-byte aligned) and fetches it with two 128-bit loads
//    and one 32-bit load; 8 lanes cover 8 consecutive pairs of one row, so a
//    wave reads 8 rows x 288 contiguous bytes per step.  The waves of a
//    workgroup split K, which keeps each wave's load count small (its
//    waits stay exact) and puts thousands of waves in flight even for
//    2560-row outputs.  Every weight load of a wave is issued before any
//    arithmetic and consumed in issue order.
//  * Each wave stages the activations of its own K slice into private LDS,
//    laid out per pair (36 dwords: 32 bf16 pairs + two block biases) so that
//    the eight columns of a wave hit distinct LDS banks.
//  * Dequantisation happens in registers without converting nibbles to
//    float: v_perm_b32 splices each nibble under the byte 0x43, which makes
//    the bf16 value 128 + nibble, and v_dot2c_f32_bf16 multiplies two of them
//    with two activations.  Per block, sum x*(128+n) - 136*sum(x) equals
//    sum x*(n-8); the -136*sum(x) bias depends on x only and is computed once
//    during staging.  The block sum is scaled by d in fp32, and the 8 lanes
//    of a row are reduced with DPP.
#include <math.h>

#include "smx_common.h"
#include "smx_launch.h"

namespace smx {
namespace {

constexpr uint32_t kNib = 0x0F0F0F0Fu;
constexpr uint32_t kMagic = 0x43434343u;   // high byte of bf16 128.0
constexpr uint32_t kSel01 = 0x04010400u;   // [b0, 0x43, b1, 0x43]
constexpr uint32_t kSel23 = 0x04030402u;   // [b2, 0x43, b3, 0x43]
constexpr uint32_t kOnes = 0x3F803F80u;    // bf16 pair (1.0, 1.0)

// acc += sum over the 8 nibbles of word w of x * (128 + nibble).
// The low nibbles of bytes (0,1) pair with activation dword xl01, bytes
// (2,3) with xl23; the high nibbles with xh01 and xh23.
__device__ __forceinline__ float word_dot(uint32_t w, uint32_t xl01, uint32_t xl23,
                                          uint32_t xh01, uint32_t xh23, float acc) {
  const uint32_t l = w & kNib;
  const uint32_t h = (w >> 4) & kNib;
  acc = dot2_bf16(perm_b32(kMagic, l, kSel01), xl01, acc);
  acc = dot2_bf16(perm_b32(kMagic, l, kSel23), xl23, acc);
  acc = dot2_bf16(perm_b32(kMagic, h, kSel01), xh01, acc);
  acc = dot2_bf16(perm_b32(kMagic, h, kSel23), xh23, acc);
  return acc;
}

struct Pair {
  u32x4 a;     // bytes 0..15  : d_even, qs_even[0..13]
  u32x4 b;     // bytes 16..31 : qs_even[14..15], d_odd, qs_odd[0..11]
  uint32_t c;  // bytes 32..35 : qs_odd[12..15]
};

__device__ __forceinline__ Pair load_pair(const uint8_t* p) {
  Pair r;
  r.a = *reinterpret_cast<const u32x4_a4*>(p);
  r.b = *reinterpret_cast<const u32x4_a4*>(p + 16);
  r.c = *reinterpret_cast<const uint32_t*>(p + 32);
  return r;
}

// A pair's staged activations in registers: its 36-dword LDS record holds
// the even block's x (16 dwords), the odd block's x (16 dwords), bias_even,
// bias_odd.
struct PairX {
  u32x4 x0, x1, x2, x3;  // even block
  u32x4 y0, y1, y2, y3;  // odd block
  u32x2 bias;
};

__device__ __forceinline__ PairX load_pair_x(const u32x4* rec) {
  return PairX{rec[0], rec[1], rec[2], rec[3], rec[4], rec[5], rec[6], rec[7],
               *reinterpret_cast<const u32x2*>(rec + 8)};
}

// Dot product of one block pair with its activations.
__device__ __forceinline__ float pair_dot(const Pair& w, const PairX& xr, float acc) {
  const u32x4 x0 = xr.x0, x1 = xr.x1, x2 = xr.x2, x3 = xr.x3;
  const u32x4 y0 = xr.y0, y1 = xr.y1, y2 = xr.y2, y3 = xr.y3;
  const u32x2 bias = xr.bias;
  // Even block: its first and last two qs bytes straddle a.x and b.x.
  const uint32_t e0 = (w.a.x & 0xffff0000u) | (w.b.x & 0x0000ffffu);  // qs 14,15,0,1
  float se = __uint_as_float(bias.x);
  se = word_dot(e0, x1.w, x0.x, x3.w, x2.x, se);     // (14,15)->x7,x15 (0,1)->x0,x8
  se = word_dot(w.a.y, x0.y, x0.z, x2.y, x2.z, se);  // (2,3)->x1,x9 (4,5)->x2,x10
  se = word_dot(w.a.z, x0.w, x1.x, x2.w, x3.x, se);  // (6,7)->x3,x11 (8,9)->x4,x12
  se = word_dot(w.a.w, x1.y, x1.z, x3.y, x3.z, se);  // (10,11)->x5,x13 (12,13)->x6,x14
  float so = __uint_as_float(bias.y);
  so = word_dot(w.b.y, y0.x, y0.y, y2.x, y2.y, so);
  so = word_dot(w.b.z, y0.z, y0.w, y2.z, y2.w, so);
  so = word_dot(w.b.w, y1.x, y1.y, y3.x, y3.y, so);
  so = word_dot(w.c, y1.z, y1.w, y3.z, y3.w, so);
  const float de = f16_bits_to_f32(w.a.x & 0xffffu);
  const float dd = f16_bits_to_f32(w.b.x >> 16);
  acc = fmaf(de, se, acc);
  acc = fmaf(dd, so, acc);
  return acc;
}

enum { EPI_STORE = 0, EPI_SWIGLU = 1, EPI_ARGMAX = 2 };

struct GemvArgs {
  const uint16_t* x;         // activation (raw input when PRO: the GEMV's own add+RMSNorm)
  const uint16_t* residual;  // PRO: added to x before the norm (may be null)
  const uint16_t* gamma;     // PRO: norm weight
  uint16_t* residual_out;    // PRO: bf16(x + residual), written by workgroup 0 (may be null)
  const uint8_t* w;
  uint16_t* y;
  uint64_t* argmax_keys;     // EPI_ARGMAX: one key per workgroup
  const uint16_t* act_lut;   // EPI_SWIGLU: null for SiLU, else the erf-GELU table (gelu_lut)
  int n_out;
  int npairs;
  int64_t up_offset_rows;
  float eps;
};

// The arguments only the epilogue (and the norm) needs, passed after the
// ones every wave needs at once: the kernel is built with kernel-argument
// preloading, which puts the leading scalar and pointer arguments in SGPRs
// before the first instruction (an aggregate is not preloaded), so the
// weight and activation loads issue without waiting for a kernarg fetch.
struct GemvTail {
  uint16_t* residual_out;
  uint16_t* y;
  uint64_t* argmax_keys;
  const uint16_t* act_lut;
  float eps;
};

// One workgroup owns RG groups of 8 weight rows.  Its waves split the K
// dimension: pair group g (pairs 8g..8g+7) belongs to wave g % ks, and lane
// 8r+c of a wave handles pair 8g+c of row r.  Each wave stages the
// activations of its own pair groups into a private LDS slice; the ks
// partial sums of a row meet in LDS at the end.
//  PRO: the staged activation is RMSNorm(x + residual) * gamma, computed in
//       the prologue (the workgroup's waves together read every element once
//       and reduce the sum of squares through LDS; workgroup 0 also writes the
//       new residual), which replaces a separate add+RMSNorm launch.
//  EPI_SWIGLU: rows 0-3 of a group are gate rows, rows 4-7 the matching up
//       rows, and the output is act(gate) * up for 4 features per group
//       (gated_act: SiLU, or erf-GELU through a table).
//  EPI_ARGMAX: besides y, each workgroup writes the max (value, -index) key
//       of its rows, for an on-device greedy argmax.
template <int NPMAX, int RG, bool PRO, int EPI>
__global__ __launch_bounds__(NPMAX <= 2 ? 1024 : 512) void q4_0_gemv_kernel(
    const uint8_t* w_, const uint16_t* x_, const uint16_t* residual_, const uint16_t* gamma_,
    int npairs_, int n_out_, int64_t up_offset_rows_, int ks_, GemvTail tail) {
  GemvArgs a;
  a.w = w_;
  a.x = x_;
  a.residual = residual_;
  a.gamma = gamma_;
  a.npairs = npairs_;
  a.n_out = n_out_;
  a.up_offset_rows = up_offset_rows_;
  a.residual_out = tail.residual_out;
  a.y = tail.y;
  a.argmax_keys = tail.argmax_keys;
  a.act_lut = tail.act_lut;
  a.eps = tail.eps;
  extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
  constexpr bool SWIGLU = EPI == EPI_SWIGLU;
  const int ks = ks_;  // waves per workgroup (blockDim.x / 64, passed to be preloaded)
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 7;
  const int rsub = lane >> 3;
  const int npairs = a.npairs;
  const int n_out = a.n_out;
  const int64_t row_bytes = (int64_t)npairs * 36;
  const int nchunks = npairs * 8;
  uint32_t* xs = lds + wave * (NPMAX * 8 * 36);
  float* part = reinterpret_cast<float*>(lds + ks * (NPMAX * 8 * 36));

  // 1. This wave's activation chunks (16 bytes each, one per lane per group).
  //    Every load of the kernel is issued unconditionally from a clamped,
  //    always-valid address and masked afterwards: a load under a divergent
  //    branch would make the compiler wait for all outstanding loads (the
  //    weights included) before the first use of the activations.
  u32x4 xv[NPMAX], rv[NPMAX], gv[NPMAX];
  bool xok[NPMAX];
  const u32x4* xg = reinterpret_cast<const u32x4*>(a.x);
  const u32x4* rgp = reinterpret_cast<const u32x4*>(PRO && a.residual ? a.residual : a.x);
#pragma unroll
  for (int t = 0; t < NPMAX; ++t) {
    const int c = (wave + ks * t) * 64 + lane;
    xok[t] = c < nchunks;
    const int cc = min(c, nchunks - 1);
    xv[t] = xg[cc];
    if constexpr (PRO) {
      rv[t] = rgp[cc];
      gv[t] = reinterpret_cast<const u32x4*>(a.gamma)[cc];
    }
  }

  // 2. The weight loads of this wave (rows past n_out and pairs past the
  //    row end read the last valid row / pair; their results are dropped).
  //    PRO with several row groups issues only the first half here and the
  //    rest after the prologue: a wave stalls at issue while the CU's memory
  //    pipeline is full of other waves' weight requests, and the prologue's
  //    barrier waits for the slowest wave, so fewer loads ahead of it end the
  //    prologue earlier while half the weights are already in flight
  //    (measured in the decode step: for norm + gate/up all loads ahead,
  //    half, or none -- half is fastest; with a single row group, and for
  //    the 9496-workgroup head, all ahead is).
  constexpr int OUT_PER_GROUP = SWIGLU ? 4 : 8;
  constexpr int GEARLY = PRO && RG > 1 && EPI != EPI_ARGMAX ? RG / 2 : RG;
  int64_t wrow[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const int o = (blockIdx.x * RG + g) * OUT_PER_GROUP + (SWIGLU ? (rsub & 3) : rsub);
    const int oc = min(o, n_out - 1);
    wrow[g] = SWIGLU ? (oc + ((rsub >> 2) ? a.up_offset_rows : 0)) : oc;
  }
  Pair wp[RG][NPMAX];
  auto load_groups = [&](int g0, int g1) {
#pragma unroll
    for (int g = g0; g < g1; ++g) {
#pragma unroll
      for (int t = 0; t < NPMAX; ++t) {
        const int j = min((wave + ks * t) * 8 + col, npairs - 1);
        wp[g][t] = load_pair(a.w + wrow[g] * row_bytes + 36 * j);
      }
    }
  };
  load_groups(0, GEARLY);
#pragma unroll
  for (int t = 0; t < NPMAX; ++t) {
    if (!xok[t]) xv[t] = u32x4{0u, 0u, 0u, 0u};
    if constexpr (PRO) {
      if (!xok[t] || !a.residual) rv[t] = u32x4{0u, 0u, 0u, 0u};
      if (!xok[t]) gv[t] = u32x4{0u, 0u, 0u, 0u};
    }
  }

  // 3. PRO: residual add + RMSNorm of the activation (norm_ub semantics:
  //    src/spark_vllm_ascend/kernels/linear.py:202-224).
  if constexpr (PRO) {
    float sv[NPMAX][8];
    float ss = 0.f;
#pragma unroll
    for (int t = 0; t < NPMAX; ++t) {
      const uint32_t xw[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
      const uint32_t rw[4] = {rv[t].x, rv[t].y, rv[t].z, rv[t].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[t][2 * i] = bf16_lo(xw[i]) + bf16_lo(rw[i]);
        sv[t][2 * i + 1] = bf16_hi(xw[i]) + bf16_hi(rw[i]);
        ss += sv[t][2 * i] * sv[t][2 * i] + sv[t][2 * i + 1] * sv[t][2 * i + 1];
      }
    }
    ss = wave_sum(ss);
    float* red = part + ks * 8 * RG;
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < ks; ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)(nchunks * 8) + a.eps);
    const bool write_res = blockIdx.x == 0 && a.residual_out;
#pragma unroll
    for (int t = 0; t < NPMAX; ++t) {
      const uint32_t gw[4] = {gv[t].x, gv[t].y, gv[t].z, gv[t].w};
      uint32_t yo[4], ro[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float s0 = sv[t][2 * i], s1 = sv[t][2 * i + 1];
        ro[i] = pack_bf16x2(s0, s1);
        yo[i] = pack_bf16x2(s0 * inv * bf16_lo(gw[i]), s1 * inv * bf16_hi(gw[i]));
      }
      xv[t] = u32x4{yo[0], yo[1], yo[2], yo[3]};
      const int c = (wave + ks * t) * 64 + lane;
      if (write_res && c < nchunks)
        st_agent(reinterpret_cast<u32x4*>(a.residual_out) + c, u32x4{ro[0], ro[1], ro[2], ro[3]});
    }
  }

  // 4. Stage the activations as 36-dword pair records with the block biases
  //    -136 * sum(x_block).  The four chunks of a block sit in one lane quad.
#pragma unroll
  for (int t = 0; t < NPMAX; ++t) {
    const u32x4 v = xv[t];
    float s = 0.f;
    s = dot2_bf16(v.x, kOnes, s);
    s = dot2_bf16(v.y, kOnes, s);
    s = dot2_bf16(v.z, kOnes, s);
    s = dot2_bf16(v.w, kOnes, s);
    s = sum4(s);
    uint32_t* rec = xs + (t * 8 + (lane >> 3)) * 36;
    *reinterpret_cast<u32x4*>(rec + 4 * (lane & 7)) = v;
    if ((lane & 3) == 0) rec[32 + ((lane >> 2) & 1)] = __float_as_uint(-136.0f * s);
  }
  load_groups(GEARLY, RG);  // the rest of the weights (PRO with RG > 1)
  // The slice is private to this wave: LDS operations of one wave complete
  // in order, so only the compiler has to be kept from reordering.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // 5. Dot products, consuming the weights in issue order.  The activation
  //    record of the lane's first pair is read from LDS before any weight is
  //    used (the scheduling barrier keeps the reads ahead of the first
  //    weight wait), so it overlaps the weight stream instead of following
  //    its last byte: graph TPOT -0.4%.  Also reading the second pair's
  //    record ahead (launches with two pair groups per lane) measured
  //    slower: the registers cost more than the overlap gains.
  const PairX first = load_pair_x(reinterpret_cast<const u32x4*>(xs + col * 36));
  __builtin_amdgcn_sched_barrier(0);
  float acc[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) acc[g] = 0.f;
#pragma unroll
  for (int t = 0; t < NPMAX; ++t) {
    const int j = (wave + ks * t) * 8 + col;
    if (j < npairs) {
      const PairX xr =
          t == 0 ? first
                 : load_pair_x(reinterpret_cast<const u32x4*>(xs + (t * 8 + col) * 36));
#pragma unroll
      for (int g = 0; g < RG; ++g) acc[g] = pair_dot(wp[g][t], xr, acc[g]);
    }
  }

  // 6. Row sums: 8 lanes by DPP, then the ks waves through LDS.
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    const float v = sum8(acc[g]);
    if (col == 0) part[wave * (8 * RG) + g * 8 + rsub] = v;
  }
  __syncthreads();
  if (wave == 0) {
    uint64_t key = 0;
    if (lane < 8 * RG) {
      const int g = lane >> 3;
      const int r = lane & 7;
      float tot = 0.f;
      for (int i = 0; i < ks; ++i) tot += part[i * (8 * RG) + lane];
      if constexpr (SWIGLU) {
        const int o = (blockIdx.x * RG + g) * 4 + r;
        if (r < 4 && o < n_out) {
          float up = 0.f;
          for (int i = 0; i < ks; ++i) up += part[i * (8 * RG) + g * 8 + r + 4];
          st_agent(a.y + o, gated_act(tot, up, a.act_lut));
        }
      } else {
        const int o = (blockIdx.x * RG + g) * 8 + r;
        if (o < n_out) {
          const uint16_t yb = f32_to_bf16(tot);
          st_agent(a.y + o, yb);
          key = ((uint64_t)bf16_order_key(yb) << 32) | (uint64_t)(0xffffffffu - (uint32_t)o);
        }
      }
    }
    if constexpr (EPI == EPI_ARGMAX) {
      for (int m = 1; m < 64; m <<= 1) {
        const uint64_t other = ((uint64_t)(uint32_t)__shfl_xor((int)(key >> 32), m, 64) << 32) |
                               (uint32_t)__shfl_xor((int)(uint32_t)key, m, 64);
        key = other > key ? other : key;
      }
      if (lane == 0) st_agent(a.argmax_keys + blockIdx.x, key);
    }
  }
  stores_done();
}

// Any k % 32 == 0 and any 2-byte alignment: one wave per output row, lanes
// stride over blocks.  Used for shapes the streaming kernel does not cover.
template <bool SWIGLU>
__global__ __launch_bounds__(64) void q4_0_gemv_generic_kernel(
    const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
    uint16_t* __restrict__ y, int n_out, int nblocks, int64_t up_offset_rows,
    const uint16_t* act_lut) {
  const int o = blockIdx.x;
  const int lane = threadIdx.x;
  const int64_t row_bytes = (int64_t)nblocks * 18;
  float acc[2] = {0.f, 0.f};
#pragma unroll
  for (int part = 0; part < (SWIGLU ? 2 : 1); ++part) {
    const int64_t row = o + (part ? up_offset_rows : 0);
    const uint16_t* wr = reinterpret_cast<const uint16_t*>(w + row * row_bytes);
    float a = 0.f;
    for (int b = lane; b < nblocks; b += 64) {
      const uint16_t* blk = wr + 9 * b;
      const float d = f16_bits_to_f32(blk[0]);
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t two = blk[1 + i];  // qs[2i], qs[2i+1]
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t byte = (two >> (8 * h)) & 0xffu;
          const int jlo = 2 * i + h;
          const float xl = bf16_bits_to_f32(x[32 * b + jlo]);
          const float xh = bf16_bits_to_f32(x[32 * b + 16 + jlo]);
          s = fmaf(xl, (float)((int)(byte & 15u) - 8), s);
          s = fmaf(xh, (float)((int)(byte >> 4) - 8), s);
        }
      }
      a = fmaf(d, s, a);
    }
    acc[part] = wave_sum(a);
  }
  if (lane == 0) {
    if constexpr (SWIGLU) {
      st_agent(y + o, gated_act(acc[0], acc[1], act_lut));
    } else {
      st_agent(y + o, f32_to_bf16(acc[0]));
    }
  }
  stores_done();
}

// One thread per block: 32 bf16 = RNE(float(d) * (nibble - 8)), exact product.
__global__ __launch_bounds__(256) void q4_0_dequant_kernel(
    const uint8_t* __restrict__ w, uint16_t* __restrict__ out, int64_t total_blocks) {
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 256 threads per workgroup
  if (b >= total_blocks) return;
  const uint16_t* blk = reinterpret_cast<const uint16_t*>(w + 18 * b);
  const float d = f16_bits_to_f32(blk[0]);
  uint32_t* o = reinterpret_cast<uint32_t*>(out + 32 * b);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t two = blk[1 + i];
    const float l0 = d * (float)((int)(two & 15u) - 8);
    const float l1 = d * (float)((int)((two >> 8) & 15u) - 8);
    const float h0 = d * (float)((int)((two >> 4) & 15u) - 8);
    const float h1 = d * (float)((int)((two >> 12) & 15u) - 8);
    st_agent(o + i, pack_bf16x2(l0, l1));
    st_agent(o + 8 + i, pack_bf16x2(h0, h1));
  }
  stores_done();
}

}  // namespace

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------

template <int NPMAX, int RG, bool PRO, int EPI>
static hipError_t launch_fast(hipStream_t s, const GemvArgs& a, int ks) {
  constexpr int OUT_PER_WG = (EPI == EPI_SWIGLU ? 4 : 8) * RG;
  const int grid = (a.n_out + OUT_PER_WG - 1) / OUT_PER_WG;
  const size_t lds = (size_t)ks * NPMAX * 8 * 36 * 4 + (size_t)ks * 8 * RG * 4 + (size_t)ks * 4;
  const GemvTail tail{a.residual_out, a.y, a.argmax_keys, a.act_lut, a.eps};
  SMX_LAUNCH((q4_0_gemv_kernel<NPMAX, RG, PRO, EPI>), dim3(grid), dim3(64 * ks), lds, s,
                     a.w, a.x, a.residual, a.gamma, a.npairs, a.n_out, a.up_offset_rows, ks,
                     tail);
  return hipGetLastError();
}

// Launch shape: rg row groups of 8 per workgroup, ks waves splitting K, np
// pair groups per wave.  Aim for a few thousand waves with balanced slices.
struct GemvShape {
  int rg, ks, np;
};

// What the GEMV fuses, as far as the launch shape goes.
enum { KIND_PLAIN = 0, KIND_NORM_STORE = 1, KIND_NORM_SWIGLU = 2, KIND_NORM_ARGMAX = 3 };

static GemvShape pick_shape(int n_out, int out_per_group, int ngroups, int kind) {
  // Measured on MI355X, in the decode step and on graph-replayed launches
  // over rotating weights:
  //  * every pair group of a row gets its own wave (np = 1) up to 16 waves
  //    per workgroup -- shorter per-wave work beats fewer, longer waves --
  //    and 17..32 pair groups take 16 waves with two groups on the first
  //    ones (2560 x 9728: 16 waves beat 10 balanced ones);
  //  * the norm-fused plain GEMV (QKV 6144 x 2560) takes two pair groups
  //    per wave: fewer waves meet at the prologue's barrier;
  //  * 16 rows per workgroup (rg = 2) above 8 pair groups (K > 4096), for
  //    very tall matrices (the 151936-row head) and for the norm + SwiGLU
  //    variant; 8 rows otherwise (6144/9728 x 2560, 2560 x 4096).
  GemvShape sh;
  const int wgs1 = (n_out + out_per_group - 1) / out_per_group;
  sh.rg = (ngroups > 8 || wgs1 >= 8192 || kind == KIND_NORM_SWIGLU) ? 2 : 1;
  if (ngroups <= 16) {
    sh.np = kind == KIND_NORM_STORE && ngroups > 2 ? 2 : 1;
    sh.ks = (ngroups + sh.np - 1) / sh.np;
  } else if (ngroups <= 32) {
    sh.np = 2;
    sh.ks = 16;
  } else {  // above 2 pair groups per lane, at most 8 waves per workgroup
    sh.np = (ngroups + 7) / 8;
    sh.ks = (ngroups + sh.np - 1) / sh.np;
  }
  // "rg,ks" overrides for tuning sweeps: SMX_GEMV_SHAPE_<n_out>_<ngroups> for
  // one shape, else SMX_GEMV_SHAPE for every shape.
  char key[64];
  snprintf(key, sizeof(key), "SMX_GEMV_SHAPE_%d_%d", n_out, ngroups);
  const char* e = tuning_env(key);
  if (!e) e = tuning_env("SMX_GEMV_SHAPE");
  if (e) {
    int a = 0, b = 0;
    if (sscanf(e, "%d,%d", &a, &b) == 2 && (a == 1 || a == 2 || a == 4) && b >= 1 && b <= 16) {
      sh.rg = a;
      sh.ks = b < ngroups ? b : ngroups;
      sh.np = (ngroups + sh.ks - 1) / sh.ks;
      if (sh.np > 2 && sh.ks > 8) {  // workgroups above 8 waves only with 1-2 pair groups
        sh.ks = 8;
        sh.np = (ngroups + 7) / 8;
      }
    }
  }
  if (sh.rg == 4 && sh.np > 2) sh.rg = 2;  // 4 row groups only with 1-2 pair groups (VGPRs)
  // The norm + argmax variant with two row groups needs more than 256 VGPRs
  // above 4 pair groups per lane (K > 16384) and would spill: one row group.
  if (kind == KIND_NORM_ARGMAX && sh.np > 4) sh.rg = 1;
  return sh;
}

template <int NPMAX, bool PRO, int EPI>
static hipError_t dispatch_rg(hipStream_t s, const GemvArgs& a, const GemvShape& sh) {
  if constexpr (NPMAX <= 2) {
    if (sh.rg == 4) return launch_fast<NPMAX, 4, PRO, EPI>(s, a, sh.ks);
  }
  // (not instantiated: the norm + argmax variant with two row groups above 4
  // pair groups per lane, which spills; pick_shape never selects it)
  if constexpr (!(PRO && EPI == EPI_ARGMAX && NPMAX > 4)) {
    if (sh.rg >= 2) return launch_fast<NPMAX, 2, PRO, EPI>(s, a, sh.ks);
  }
  return launch_fast<NPMAX, 1, PRO, EPI>(s, a, sh.ks);
}

template <bool PRO, int EPI>
static hipError_t dispatch_np(hipStream_t s, const GemvArgs& a, const GemvShape& sh) {
  switch (sh.np) {
    case 1: return dispatch_rg<1, PRO, EPI>(s, a, sh);
    case 2: return dispatch_rg<2, PRO, EPI>(s, a, sh);
    case 3: return dispatch_rg<3, PRO, EPI>(s, a, sh);
    case 4: return dispatch_rg<4, PRO, EPI>(s, a, sh);
    case 5: return dispatch_rg<5, PRO, EPI>(s, a, sh);
    case 6: return dispatch_rg<6, PRO, EPI>(s, a, sh);
    case 7: return dispatch_rg<7, PRO, EPI>(s, a, sh);
    case 8: return dispatch_rg<8, PRO, EPI>(s, a, sh);
    default: return hipErrorInvalidValue;
  }
}

// Whether the streaming kernel takes this call (else the generic kernel).
static bool fast_path(int64_t k, const void* x, const void* w, GemvShape* sh, int64_t n_out,
                      int out_per_group, int kind = KIND_PLAIN) {
  if (k % 64 != 0 || (uintptr_t)w % 4 != 0 || (uintptr_t)x % 16 != 0) return false;
  const int ngroups = (int)((k / 64 + 7) / 8);
  *sh = pick_shape((int)n_out, out_per_group, ngroups, kind);
  return sh->np <= 8;
}

// Grid size of the streaming kernel for an argmax GEMV (keys written).
static int64_t argmax_workgroups(int64_t n, int64_t k, const void* x, const void* w) {
  GemvShape sh;
  if (!fast_path(k, x, w, &sh, n, 8, KIND_NORM_ARGMAX)) return -1;
  return (n + 8 * sh.rg - 1) / (8 * sh.rg);
}

static hipError_t gemv_dispatch(hipStream_t s, GemvArgs a, int64_t k, int epi, bool pro) {
  const int64_t nblocks = k / 32;
  a.npairs = (int)(nblocks / 2);
  GemvShape sh{1, 1, 1};
  const int kind = !pro ? KIND_PLAIN
                   : epi == EPI_SWIGLU ? KIND_NORM_SWIGLU
                   : epi == EPI_STORE ? KIND_NORM_STORE
                                      : KIND_NORM_ARGMAX;
  if (!fast_path(k, a.x, a.w, &sh, a.n_out, epi == EPI_SWIGLU ? 4 : 8, kind)) {
    if (pro || epi == EPI_ARGMAX) return hipErrorInvalidValue;  // callers check first
    if (epi == EPI_SWIGLU)
      SMX_LAUNCH(q4_0_gemv_generic_kernel<true>, dim3((unsigned)a.n_out), dim3(64), 0, s,
                         a.x, a.w, a.y, a.n_out, (int)nblocks, a.up_offset_rows, a.act_lut);
    else
      SMX_LAUNCH(q4_0_gemv_generic_kernel<false>, dim3((unsigned)a.n_out), dim3(64), 0,
                         s, a.x, a.w, a.y, a.n_out, (int)nblocks, a.up_offset_rows, a.act_lut);
    return hipGetLastError();
  }
  if (pro) {
    if (epi == EPI_SWIGLU) return dispatch_np<true, EPI_SWIGLU>(s, a, sh);
    if (epi == EPI_ARGMAX) return dispatch_np<true, EPI_ARGMAX>(s, a, sh);
    return dispatch_np<true, EPI_STORE>(s, a, sh);
  }
  if (epi == EPI_SWIGLU) return dispatch_np<false, EPI_SWIGLU>(s, a, sh);
  if (epi == EPI_ARGMAX) return dispatch_np<false, EPI_ARGMAX>(s, a, sh);
  return dispatch_np<false, EPI_STORE>(s, a, sh);
}

}  // namespace smx

#include "smx_abi_util.h"

extern "C" int smx_q4_0_dequant_bf16(void* stream, const void* w, void* out, int64_t n,
                                     int64_t k) {
  SMX_REQUIRE(w && out, "w and out must be non-null");
  SMX_REQUIRE(n >= 1 && k >= 32 && k % 32 == 0, "need n >= 1 and k a positive multiple of 32");
  SMX_REQUIRE((uintptr_t)w % 2 == 0, "w must be 2-byte aligned");
  SMX_REQUIRE((uintptr_t)out % 4 == 0, "out must be 4-byte aligned");
  const int64_t total = n * (k / 32);
  const int64_t grid = (total + 255) / 256;
  SMX_REQUIRE(grid < (1ll << 31), "tensor too large");
  SMX_LAUNCH(smx::q4_0_dequant_kernel, dim3((unsigned)grid), dim3(256), 0,
                     (hipStream_t)stream, (const uint8_t*)w, (uint16_t*)out, total);
  return (int)hipGetLastError();
}

static smx::GemvArgs plain_args(const void* x, const void* w, void* y, int64_t n) {
  smx::GemvArgs a{};
  a.x = (const uint16_t*)x;
  a.w = (const uint8_t*)w;
  a.y = (uint16_t*)y;
  a.n_out = (int)n;
  return a;
}

extern "C" int smx_q4_0_gemv(void* stream, const void* x, const void* w, void* y, int64_t n,
                             int64_t k) {
  SMX_REQUIRE(x && w && y, "x, w and y must be non-null");
  SMX_REQUIRE(n >= 1 && n < (1ll << 31), "n out of range");
  SMX_REQUIRE(k >= 32 && k % 32 == 0 && k <= (1 << 20), "k must be a multiple of 32 in [32, 2^20]");
  SMX_REQUIRE((uintptr_t)x % 2 == 0 && (uintptr_t)w % 2 == 0 && (uintptr_t)y % 2 == 0,
              "x, w and y must be 2-byte aligned");
  return (int)smx::gemv_dispatch((hipStream_t)stream, plain_args(x, w, y, n), k, smx::EPI_STORE,
                                 false);
}

// Shared checks of the gated (gate/up) GEMV entries.
#define SMX_GATED_GEMV_CHECKS                                                                    \
  SMX_REQUIRE(x && w && out, "x, w and out must be non-null");                                   \
  SMX_REQUIRE(d >= 1 && d < (1ll << 30), "d out of range");                                      \
  SMX_REQUIRE(k >= 32 && k % 32 == 0 && k <= (1 << 20), "k must be a multiple of 32 in [32, 2^20]"); \
  SMX_REQUIRE((uintptr_t)x % 2 == 0 && (uintptr_t)w % 2 == 0 && (uintptr_t)out % 2 == 0,         \
              "x, w and out must be 2-byte aligned")

static int gemv_gated(void* stream, const void* x, const void* w, const void* lut, void* out,
                      int64_t d, int64_t k) {
  smx::GemvArgs a = plain_args(x, w, out, d);
  a.up_offset_rows = d;
  a.act_lut = (const uint16_t*)lut;
  return (int)smx::gemv_dispatch((hipStream_t)stream, a, k, smx::EPI_SWIGLU, false);
}

extern "C" int smx_q4_0_gemv_swiglu(void* stream, const void* x, const void* w, void* out,
                                    int64_t d, int64_t k) {
  SMX_GATED_GEMV_CHECKS;
  return gemv_gated(stream, x, w, nullptr, out, d, k);
}

extern "C" int smx_q4_0_gemv_gelu(void* stream, const void* x, const void* w, const void* lut,
                                  void* out, int64_t d, int64_t k) {
  SMX_GATED_GEMV_CHECKS;
  SMX_REQUIRE(lut && (uintptr_t)lut % 2 == 0, "lut must be non-null and 2-byte aligned");
  return gemv_gated(stream, x, w, lut, out, d, k);
}

// Shared checks of the entries with the add+RMSNorm prologue.
#define SMX_NORM_GEMV_CHECKS(X, W, OUT, N)                                                       \
  SMX_REQUIRE(X && gamma && W && OUT, "x, gamma, w and the output must be non-null");           \
  SMX_REQUIRE(N >= 1 && N < (1ll << 30), "output size out of range");                           \
  SMX_REQUIRE(k >= 64 && k % 64 == 0 && k <= 65536, "k must be a multiple of 64 in [64, 65536]"); \
  SMX_REQUIRE(eps >= 0.f && std::isfinite(eps), "eps must be finite and >= 0");                 \
  SMX_REQUIRE((uintptr_t)X % 16 == 0 && (uintptr_t)gamma % 16 == 0 &&                            \
                  (uintptr_t)residual % 16 == 0 && (uintptr_t)residual_out % 16 == 0 &&         \
                  (uintptr_t)W % 4 == 0 && (uintptr_t)OUT % 2 == 0,                              \
              "x, residual, gamma, residual_out 16-byte aligned; w 4-byte aligned");             \
  SMX_REQUIRE(!residual_out || (residual_out != residual && residual_out != X),                  \
              "residual_out must not alias x or residual");                                      \
  {                                                                                              \
    smx::GemvShape sh_;                                                                          \
    SMX_REQUIRE(smx::fast_path(k, X, W, &sh_, N, 8), "shape not supported by the fused kernel");  \
  }

static smx::GemvArgs norm_args(const void* x, const void* residual, const void* gamma,
                               void* residual_out, const void* w, void* y, int64_t n,
                               float eps) {
  smx::GemvArgs a = plain_args(x, w, y, n);
  a.residual = (const uint16_t*)residual;
  a.gamma = (const uint16_t*)gamma;
  a.residual_out = (uint16_t*)residual_out;
  a.eps = eps;
  return a;
}

extern "C" int smx_q4_0_add_rmsnorm_gemv(void* stream, const void* x, const void* residual,
                                         const void* gamma, void* residual_out, const void* w,
                                         void* y, int64_t n, int64_t k, float eps) {
  SMX_NORM_GEMV_CHECKS(x, w, y, n);
  return (int)smx::gemv_dispatch(
      (hipStream_t)stream, norm_args(x, residual, gamma, residual_out, w, y, n, eps), k,
      smx::EPI_STORE, true);
}

static int norm_gemv_gated(void* stream, const void* x, const void* residual, const void* gamma,
                           void* residual_out, const void* w, const void* lut, void* out,
                           int64_t d, int64_t k, float eps) {
  smx::GemvArgs a = norm_args(x, residual, gamma, residual_out, w, out, d, eps);
  a.up_offset_rows = d;
  a.act_lut = (const uint16_t*)lut;
  return (int)smx::gemv_dispatch((hipStream_t)stream, a, k, smx::EPI_SWIGLU, true);
}

extern "C" int smx_q4_0_add_rmsnorm_gemv_swiglu(void* stream, const void* x, const void* residual,
                                                const void* gamma, void* residual_out,
                                                const void* w, void* out, int64_t d, int64_t k,
                                                float eps) {
  SMX_NORM_GEMV_CHECKS(x, w, out, d);
  return norm_gemv_gated(stream, x, residual, gamma, residual_out, w, nullptr, out, d, k, eps);
}

extern "C" int smx_q4_0_add_rmsnorm_gemv_gelu(void* stream, const void* x, const void* residual,
                                              const void* gamma, void* residual_out,
                                              const void* w, const void* lut, void* out,
                                              int64_t d, int64_t k, float eps) {
  SMX_NORM_GEMV_CHECKS(x, w, out, d);
  SMX_REQUIRE(lut && (uintptr_t)lut % 2 == 0, "lut must be non-null and 2-byte aligned");
  return norm_gemv_gated(stream, x, residual, gamma, residual_out, w, lut, out, d, k, eps);
}

extern "C" int64_t smx_q4_0_argmax_keys_size(int64_t n, int64_t k) {
  if (n < 1 || k < 64 || k % 64) return -1;
  static const uint16_t dummy[8] __attribute__((aligned(16))) = {};
  return smx::argmax_workgroups(n, k, dummy, dummy);
}

extern "C" int smx_q4_0_add_rmsnorm_gemv_argmax(void* stream, const void* x,
                                                const void* residual, const void* gamma,
                                                const void* w, void* logits, uint64_t* keys,
                                                int64_t num_keys, int64_t n, int64_t k,
                                                float eps) {
  void* residual_out = nullptr;
  SMX_NORM_GEMV_CHECKS(x, w, logits, n);
  SMX_REQUIRE(keys && (uintptr_t)keys % 8 == 0, "keys must be non-null and 8-byte aligned");
  SMX_REQUIRE(num_keys == smx::argmax_workgroups(n, k, x, w),
              "num_keys must equal smx_q4_0_argmax_keys_size(n, k)");
  smx::GemvArgs a = norm_args(x, residual, gamma, nullptr, w, logits, n, eps);
  a.argmax_keys = keys;
  return (int)smx::gemv_dispatch((hipStream_t)stream, a, k, smx::EPI_ARGMAX, true);
}
