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
// head against ~2k flops):
//  * one workgroup (4 or 8 waves) per (split, kv head, sequence); the
//    split's tokens are cut into contiguous 32-aligned chunks, one per wave;
//  * a wave walks its chunk in 32-token tiles, pipelined in place: the next
//    tile's K and V loads are in flight while the current tile is computed;
//  * QK: 4 lanes per token, each owning 32 of the 128 dims for all 4 GQA
//    heads (q lives in registers as bf16 pairs); v_dot2c_f32_bf16 + a quad
//    reduction give the 4 scores;
//  * PV: 16 lanes per token, each owning 8 dims; two tokens' V values are
//    spliced into bf16 pairs with v_perm_b32 and meet the matching pair of
//    bf16 probabilities (staged through LDS) in v_dot2c_f32_bf16;
//  * the 4 waves' (max, sum, O) states are combined through LDS.
#include <math.h>

#include "smx_common.h"

namespace smx {
namespace {

constexpr int HD = 128;
constexpr int G = 4;       // q heads per kv head
constexpr int TILE = 32;   // tokens per wave iteration

template <int CTRL>
__device__ __forceinline__ float dppf(float v) { return dpp_f32<CTRL>(v); }
constexpr int DPP_ROW_ROR4 = 0x124;
constexpr int DPP_ROW_ROR8 = 0x128;

// max over the 16 lane quads of a wave (values replicated inside a quad)
__device__ __forceinline__ float quad_max_wave(float v) {
  v = fmaxf(v, dppf<DPP_ROW_ROR4>(v));
  v = fmaxf(v, dppf<DPP_ROW_ROR8>(v));
  v = fmaxf(v, shfl_xor_f32(v, 16));
  v = fmaxf(v, shfl_xor_f32(v, 32));
  return v;
}
// sum over the 16 lanes of a wave that share lane & 3
__device__ __forceinline__ float sum_stride4(float v) {
  v += dppf<DPP_ROW_ROR4>(v);
  v += dppf<DPP_ROW_ROR8>(v);
  v += shfl_xor_f32(v, 16);
  v += shfl_xor_f32(v, 32);
  return v;
}

// WAVES waves per workgroup; the split's tokens are cut into WAVES
// contiguous 32-aligned chunks.  Within a wave, tiles are software-pipelined
// in place: the next tile's K loads are issued as soon as the current K has
// been consumed by QK, and its V loads as soon as PV has consumed V, so one
// tile of registers keeps a load in flight during all arithmetic.
template <int WAVES>
__global__ __launch_bounds__(64 * WAVES) void splitkv_decode_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ block_table,
    const int32_t* __restrict__ seq_lens, float* __restrict__ part_o,
    float* __restrict__ part_lse, int num_splits, int max_blocks, int num_blocks, int bs_log2,
    int n_q, int n_kv, float scale_log2) {
  constexpr int NT = 64 * WAVES;
  __shared__ uint32_t p2[WAVES][64];        // per wave: [jp][vt][h] bf16 probability pairs
  __shared__ float o_w[WAVES][G * HD];       // per wave O (unnormalised)
  __shared__ float m_w[WAVES][G], l_w[WAVES][G];
  __shared__ int bad_w[WAVES];

  const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // A length beyond the block table is clamped to what the table can address.
  const int L = min(seq_lens[seq], max_blocks << bs_log2);
  const int tps = ((L + num_splits - 1) / num_splits + TILE - 1) / TILE * TILE;
  const int s0 = split * tps;
  const int s1 = min(L, s0 + tps);
  float* po = part_o + (((int64_t)seq * num_splits + split) * n_q + kvh * G) * HD;
  float* pl = part_lse + ((int64_t)seq * num_splits + split) * n_q + kvh * G;
  if (s0 >= s1) {
    for (int i = tid; i < G * HD; i += NT) po[i] = 0.f;
    if (tid < G) pl[tid] = -INFINITY;
    return;
  }
  const int len = s1 - s0;
  const int wlen = ((len + WAVES - 1) / WAVES + TILE - 1) / TILE * TILE;
  const int w0 = s0 + wave * wlen;
  const int w1 = min(s1, w0 + wlen);

  const int bs = 1 << bs_log2;
  const int64_t tok_stride = (int64_t)n_kv * HD;
  const int64_t page_stride = tok_stride << bs_log2;
  const int32_t* bt = block_table + (int64_t)seq * max_blocks;

  // lane roles
  const int qd = lane >> 2, dq = lane & 3;   // QK: token slot, 32-dim slice
  const int vt = lane >> 4, dv = lane & 15;  // PV: token slot, 8-dim slice

  // q for the 4 heads of this group, dims 32*dq .. 32*dq+31
  u32x4 qr[G][4];
  {
    const uint16_t* qb = q + ((int64_t)seq * n_q + kvh * G) * HD + 32 * dq;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) qr[h][i] = *reinterpret_cast<const u32x4*>(qb + h * HD + 8 * i);
  }

  // A block-table entry outside [0, num_blocks) is never dereferenced: the
  // page is replaced by page 0 and the partial is poisoned with NaN below.
  bool bad_page = false;
  auto page_of = [&](int t0) -> int64_t {
    int pg = bt[t0 >> bs_log2];
    if ((unsigned)pg >= (unsigned)num_blocks) {
      bad_page = true;
      pg = 0;
    }
    return (int64_t)pg * page_stride + (int64_t)(t0 & (bs - 1)) * tok_stride + kvh * HD;
  };
  u32x4 kr[2][4];  // QK rounds 0/1: dims 32*dq .. 32*dq+31 of token t0 + 16*rr + qd
  u32x4 vr[4][2];  // PV pairs jp: tokens t0 + 8jp + vt (+4), dims 8*dv .. 8*dv+7
  // Tokens past the chunk end are loaded from the tile's first token (always
  // valid) instead of branching; their scores are masked to -inf, so their
  // probabilities are exactly 0.
  auto load_k = [&](int t0, int64_t base) {
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int t = rr * 16 + qd;
      const int te = t0 + t < w1 ? t : 0;
      const uint16_t* p = kc + base + te * tok_stride + 32 * dq;
#pragma unroll
      for (int i = 0; i < 4; ++i) kr[rr][i] = *reinterpret_cast<const u32x4*>(p + 8 * i);
    }
  };
  auto load_v = [&](int t0, int64_t base) {
#pragma unroll
    for (int jp = 0; jp < 4; ++jp)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int t = 8 * jp + vt + 4 * hf;
        const int te = t0 + t < w1 ? t : 0;
        vr[jp][hf] = *reinterpret_cast<const u32x4*>(vc + base + te * tok_stride + 8 * dv);
      }
  };

  float m[G];
  float o[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[h][i] = 0.f;
  }
  float l_lane = 0.f;  // running sum for head dq over this lane's tokens

  if (w0 < w1) {
    const int64_t b0 = page_of(w0);
    load_k(w0, b0);
    load_v(w0, b0);
  }
  for (int t0 = w0; t0 < w1; t0 += TILE) {
    const bool more = t0 + TILE < w1;
    const int64_t bnext = more ? page_of(t0 + TILE) : 0;

    // ---- scores for the two QK rounds (tokens t0 + 16*rr + qd)
    float s[2][G];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a = dot2_bf16(qr[h][i].x, kr[rr][i].x, a);
          a = dot2_bf16(qr[h][i].y, kr[rr][i].y, a);
          a = dot2_bf16(qr[h][i].z, kr[rr][i].z, a);
          a = dot2_bf16(qr[h][i].w, kr[rr][i].w, a);
        }
        a = sum4(a) * scale_log2;
        s[rr][h] = (t0 + rr * 16 + qd < w1) ? a : -INFINITY;
      }
    }
    if (more) load_k(t0 + TILE, bnext);

    // ---- online softmax update (log2 domain)
    float alpha[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float tmax = quad_max_wave(fmaxf(s[0][h], s[1][h]));
      const float mn = fmaxf(m[h], tmax);
      alpha[h] = exp2f(m[h] - mn);
      m[h] = mn;
    }
    const float my_m = dq == 0 ? m[0] : dq == 1 ? m[1] : dq == 2 ? m[2] : m[3];
    const float my_alpha = dq == 0 ? alpha[0] : dq == 1 ? alpha[1] : dq == 2 ? alpha[2] : alpha[3];
    float p_sum = 0.f;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const float sv = dq == 0 ? s[rr][0] : dq == 1 ? s[rr][1] : dq == 2 ? s[rr][2] : s[rr][3];
      const float p = exp2f(sv - my_m);
      p_sum += p;
      const int t = rr * 16 + qd;  // tile-relative token
      const int jp = t >> 3, within = t & 7;
      uint16_t* dst = reinterpret_cast<uint16_t*>(&p2[wave][(jp * 4 + (within & 3)) * 4 + dq]);
      dst[within >> 2] = f32_to_bf16(p);
    }
    l_lane = l_lane * my_alpha + p_sum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- O = O * alpha + P V
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) o[h][i] *= alpha[h];
#pragma unroll
    for (int jp = 0; jp < 4; ++jp) {
      const u32x4 pp = *reinterpret_cast<const u32x4*>(&p2[wave][(jp * 4 + vt) * 4]);
      const u32x4 va = vr[jp][0], vb2 = vr[jp][1];
      uint32_t vpair[8];  // (v[t1][d], v[t2][d]) for the 8 dims
      vpair[0] = perm_b32(vb2.x, va.x, 0x05040100u);
      vpair[1] = perm_b32(vb2.x, va.x, 0x07060302u);
      vpair[2] = perm_b32(vb2.y, va.y, 0x05040100u);
      vpair[3] = perm_b32(vb2.y, va.y, 0x07060302u);
      vpair[4] = perm_b32(vb2.z, va.z, 0x05040100u);
      vpair[5] = perm_b32(vb2.z, va.z, 0x07060302u);
      vpair[6] = perm_b32(vb2.w, va.w, 0x05040100u);
      vpair[7] = perm_b32(vb2.w, va.w, 0x07060302u);
      const uint32_t ph[G] = {pp.x, pp.y, pp.z, pp.w};
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int i = 0; i < 8; ++i) o[h][i] = dot2_bf16(ph[h], vpair[i], o[h][i]);
    }
    if (more) load_v(t0 + TILE, bnext);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- per-wave state to LDS
  const float l_tot = sum_stride4(l_lane);
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = o[h][i];
      v += shfl_xor_f32(v, 16);
      v += shfl_xor_f32(v, 32);
      o[h][i] = v;
    }
  if (vt == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) o_w[wave][h * HD + 8 * dv + i] = o[h][i];
  }
  if (lane == 0) bad_w[wave] = bad_page ? 1 : 0;
  if (lane < G) {
    l_w[wave][lane] = l_tot;
    m_w[wave][lane] = lane == 0 ? m[0] : lane == 1 ? m[1] : lane == 2 ? m[2] : m[3];
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
    po[e] = bad ? __builtin_nanf("") : ot / lt;
    if ((e % HD) == 0) pl[h] = bad ? __builtin_nanf("") : (mt + log2f(lt)) * 0.69314718055994530942f;
  }
}

// One workgroup per (q head, sequence); one thread per head dim.
__global__ __launch_bounds__(128) void lse_merge_kernel(const float* __restrict__ part_o,
                                                        const float* __restrict__ part_lse,
                                                        uint16_t* __restrict__ out,
                                                        int num_splits, int n_q, int hd) {
  const int h = blockIdx.x, seq = blockIdx.y;
  const float* lse = part_lse + (int64_t)seq * num_splits * n_q + h;
  float mx = -INFINITY;
  for (int s = 0; s < num_splits; ++s) mx = fmaxf(mx, lse[(int64_t)s * n_q]);
  float den = 0.f;
  for (int s = 0; s < num_splits; ++s) {
    const float v = lse[(int64_t)s * n_q];
    den += v == -INFINITY ? 0.f : expf(v - mx);
  }
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.f;
    for (int s = 0; s < num_splits; ++s) {
      const float v = lse[(int64_t)s * n_q];
      if (v == -INFINITY) continue;
      const float wgt = expf(v - mx) / den;
      acc += part_o[(((int64_t)seq * num_splits + s) * n_q + h) * hd + d] * wgt;
    }
    out[((int64_t)seq * n_q + h) * hd + d] = f32_to_bf16(acc);
  }
}

}  // namespace
}  // namespace smx

#include "smx_abi_util.h"

extern "C" int smx_splitkv_decode(void* stream, const void* q, const void* k_cache,
                                  const void* v_cache, const int32_t* block_table,
                                  const int32_t* seq_lens, float* partial_o, float* partial_lse,
                                  int32_t num_seqs, int32_t num_splits, int32_t max_blocks,
                                  int32_t num_blocks, int32_t block_size, int32_t n_q,
                                  int32_t n_kv, int32_t head_dim, float scale) {
  SMX_REQUIRE(q && k_cache && v_cache && block_table && seq_lens && partial_o && partial_lse,
              "null pointer argument");
  SMX_REQUIRE(num_seqs >= 1 && num_seqs <= 65535, "num_seqs must be in [1, 65535]");
  SMX_REQUIRE(num_splits >= 1 && num_splits <= 4096, "num_splits must be in [1, 4096]");
  SMX_REQUIRE(max_blocks >= 1 && num_blocks >= 1, "max_blocks and num_blocks must be >= 1");
  SMX_REQUIRE(head_dim == 128, "head_dim must be 128");
  SMX_REQUIRE(n_kv >= 1 && n_q == 4 * n_kv && n_kv <= 65535, "need n_q == 4 * n_kv (GQA 4:1)");
  SMX_REQUIRE(block_size >= 32 && block_size <= 4096 && (block_size & (block_size - 1)) == 0,
              "block_size must be a power of two in [32, 4096]");
  SMX_REQUIRE(scale > 0.f && isfinite(scale), "scale must be positive and finite");
  SMX_REQUIRE((uintptr_t)q % 16 == 0 && (uintptr_t)k_cache % 16 == 0 &&
                  (uintptr_t)v_cache % 16 == 0 && (uintptr_t)block_table % 4 == 0 &&
                  (uintptr_t)seq_lens % 4 == 0 && (uintptr_t)partial_o % 4 == 0 &&
                  (uintptr_t)partial_lse % 4 == 0,
              "q, k_cache and v_cache must be 16-byte aligned; int/float arrays 4-byte aligned");
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  const float scale_log2 = scale * 1.44269504088896340736f;
  int waves = 4;
  const char* e = getenv("SMX_ATTN_WAVES");  // 4 or 8 waves per workgroup, for tuning sweeps
  if (e && atoi(e) == 8) waves = 8;
  if (waves == 8)
    hipLaunchKernelGGL(smx::splitkv_decode_kernel<8>, dim3(num_splits, n_kv, num_seqs), dim3(512),
                       0, (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k_cache,
                       (const uint16_t*)v_cache, block_table, seq_lens, partial_o, partial_lse,
                       num_splits, max_blocks, num_blocks, bs_log2, n_q, n_kv, scale_log2);
  else
    hipLaunchKernelGGL(smx::splitkv_decode_kernel<4>, dim3(num_splits, n_kv, num_seqs), dim3(256),
                       0, (hipStream_t)stream, (const uint16_t*)q, (const uint16_t*)k_cache,
                       (const uint16_t*)v_cache, block_table, seq_lens, partial_o, partial_lse,
                       num_splits, max_blocks, num_blocks, bs_log2, n_q, n_kv, scale_log2);
  return (int)hipGetLastError();
}

extern "C" int smx_lse_merge(void* stream, const float* partial_o, const float* partial_lse,
                             void* out, int32_t num_seqs, int32_t num_splits, int32_t n_q,
                             int32_t head_dim) {
  SMX_REQUIRE(partial_o && partial_lse && out, "null pointer argument");
  SMX_REQUIRE(num_seqs >= 1 && num_seqs <= 65535, "num_seqs must be in [1, 65535]");
  SMX_REQUIRE(num_splits >= 1 && num_splits <= 4096, "num_splits must be in [1, 4096]");
  SMX_REQUIRE(n_q >= 1 && head_dim >= 1 && head_dim <= 1024, "bad n_q or head_dim");
  SMX_REQUIRE((uintptr_t)out % 2 == 0 && (uintptr_t)partial_o % 4 == 0 &&
                  (uintptr_t)partial_lse % 4 == 0,
              "misaligned pointer");
  hipLaunchKernelGGL(smx::lse_merge_kernel, dim3(n_q, num_seqs), dim3(128), 0,
                     (hipStream_t)stream, partial_o, partial_lse, (uint16_t*)out, num_splits,
                     n_q, head_dim);
  return (int)hipGetLastError();
}
