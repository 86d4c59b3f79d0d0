// Q4_0 GEMM for a few activation rows (batched decode, M <= 16) on MFMA.
//
// Y[m][n] = sum_k X[m][k] * W[n][k] with W in GGUF Q4_0 blocks (fp16 d, 16
// bytes of nibbles, value d * (nibble - 8)), bf16 X and Y, fp32 accumulation
// -- the GEMV semantics of src/spark_vllm_ascend/kernels/linear.py:16-200 for
// several rows at once (the reference runs batch 1 only).
//
// Both kernels put 16 weight rows x 32 k on one v_mfma_f32_16x16x32_bf16
// (A = the activation rows as the M side, B = W^T), with the weights as bf16
// 128 + nibble (v_perm_b32 splices each nibble under the byte 0x43), a second
// MFMA against a constant -136 operand (C = A.B(128+n) + A.B(-136) = sum x (n - 8),
// no per-block activation sums) and the block result scaled by the row's fp16
// d in fp32.
//  * q4_0_gemm_tile_kernel (16-byte aligned activations): the GEMV's 16-byte
//    pair loads, redistributed across lanes by permlane swaps (below).
//  * q4_0_gemm_kernel (8-byte aligned activations): one workgroup of 8 waves
//    per 16 rows, each lane loading one 32-bit word of a block's nibbles.
//    A lane holds weight row n = l & 15 and k-slot group g = l >> 4.  The K
//    order inside an MFMA is a permutation shared by A and B: slot j of group
//    g is the element of the word's byte j & 3, low nibble for j < 4 and high
//    nibble (element + 16) otherwise.  Block pairs are 36 bytes, so the even
//    block's nibbles start 2 bytes into a dword; its group-0 word is spliced
//    from the pair's dwords 0 and 4 (elements 14, 15, 0, 1).
#include "smx_common.h"
#include "smx_launch.h"

namespace smx {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kNibG = 0x0F0F0F0Fu;
constexpr uint32_t kMagicG = 0x43434343u;
constexpr uint32_t kSel01G = 0x04010400u;  // [b0, 0x43, b1, 0x43]
constexpr uint32_t kSel23G = 0x04030402u;  // [b2, 0x43, b3, 0x43]
constexpr uint32_t kNeg136 = 0xC308C308u;  // bf16 pair (-136, -136)

struct GemmArgs {
  const uint16_t* x;  // [m, k] bf16, row stride ldx elements
  const uint8_t* w;   // Q4_0 blocks, row stride npairs * 36 bytes
  uint16_t* y;        // [m, ldy] bf16
  int m, n_out, npairs;
  int64_t ldx, ldy, up_offset_rows;
  const uint16_t* act_lut;  // SWIGLU: null for SiLU, else the erf-GELU table (gelu_lut)
};

__device__ __forceinline__ bf16x8 dequant_word(uint32_t w) {
  const uint32_t l = w & kNibG, h = (w >> 4) & kNibG;
  uint32_t r[4] = {perm_b32(kMagicG, l, kSel01G), perm_b32(kMagicG, l, kSel23G),
                   perm_b32(kMagicG, h, kSel01G), perm_b32(kMagicG, h, kSel23G)};
  return __builtin_bit_cast(bf16x8, r);
}

template <bool SWIGLU>
__global__ __launch_bounds__(512) void q4_0_gemm_kernel(GemmArgs a) {
  constexpr int WAVES = 8, CH = 8;  // pairs per wave per round of loads
  __shared__ f32x4 red[WAVES][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  // This lane's weight row: plain, 16 rows per tile; SwiGLU, 8 gate rows
  // then the 8 matching up rows.
  int wrow;
  if constexpr (SWIGLU) {
    const int f = min(blockIdx.x * 8 + (n & 7), a.n_out - 1);
    wrow = f + (n >= 8 ? (int)a.up_offset_rows : 0);
  } else {
    wrow = min(blockIdx.x * 16 + n, a.n_out - 1);
  }
  const uint32_t* wr = reinterpret_cast<const uint32_t*>(a.w + (int64_t)wrow * a.npairs * 36);
  // This lane's activation row (A side) and its element offsets per block.
  const bool m_ok = n < a.m;
  const uint32_t* xr = reinterpret_cast<const uint32_t*>(a.x + (int64_t)min(n, a.m - 1) * a.ldx);
  const int e0 = g == 0 ? 14 : 4 * g - 2, e1 = g == 0 ? 0 : 4 * g;  // even block
  const int o0 = 4 * g;                                              // odd block
  bf16x8 bneg;
  {
    const uint32_t c[4] = {kNeg136, kNeg136, kNeg136, kNeg136};
    bneg = __builtin_bit_cast(bf16x8, c);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = zero;
  for (int p0 = wave; p0 < a.npairs; p0 += WAVES * CH) {
    uint32_t d0[CH], d4[CH], de[CH], dd[CH];
    uint32_t xe[CH][4];
    u32x2_t xo[CH][2];
    // every load of the round first (clamped to valid pairs)
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      const int p = min(p0 + WAVES * t, a.npairs - 1);
      const uint32_t* pw = wr + 9 * p;
      d0[t] = pw[0];
      d4[t] = pw[4];
      de[t] = pw[g];
      dd[t] = pw[5 + g];
      const uint32_t* xb = xr + 32 * p;  // 64 elements = 32 dwords per pair
      xe[t][0] = xb[e0 / 2];
      xe[t][1] = xb[e1 / 2];
      xe[t][2] = xb[(e0 + 16) / 2];
      xe[t][3] = xb[(e1 + 16) / 2];
      xo[t][0] = *reinterpret_cast<const u32x2_t*>(xb + 16 + o0 / 2);
      xo[t][1] = *reinterpret_cast<const u32x2_t*>(xb + 16 + (o0 + 16) / 2);
    }
    // Branch-free: a pair past the row end is computed on the clamped pair
    // and dropped, so the loads above stay ahead of all the arithmetic.
#pragma unroll
    for (int t = 0; t < CH; ++t) {
      const bool valid = p0 + WAVES * t < a.npairs;
      const uint32_t we = g == 0 ? ((d0[t] & 0xffff0000u) | (d4[t] & 0x0000ffffu)) : de[t];
      uint32_t ae[4] = {xe[t][0], xe[t][1], xe[t][2], xe[t][3]};
      uint32_t ao[4] = {xo[t][0].x, xo[t][0].y, xo[t][1].x, xo[t][1].y};
      if (!m_ok) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ae[i] = ao[i] = 0u;
      }
      const bf16x8 A_e = __builtin_bit_cast(bf16x8, ae), A_o = __builtin_bit_cast(bf16x8, ao);
      f32x4 ce = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A_e, dequant_word(we), zero, 0, 0, 0);
      ce = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A_e, bneg, ce, 0, 0, 0);
      f32x4 co = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A_o, dequant_word(dd[t]), zero, 0, 0, 0);
      co = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A_o, bneg, co, 0, 0, 0);
      const float sde = f16_bits_to_f32(d0[t] & 0xffffu);
      const float sdo = f16_bits_to_f32(d4[t] >> 16);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = fmaf(sdo, co[r], fmaf(sde, ce[r], acc[r]));
        acc[r] = valid ? v : acc[r];
      }
    }
  }
  // C layout: lane l holds rows m = 4 (l >> 4) + r of column n = l & 15.
  red[wave][lane] = acc;
  __syncthreads();
  const int tid = threadIdx.x;
  if (tid < 256) {
    const int m = tid >> 4, nn = tid & 15;
    auto total = [&](int col) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) s += red[w][16 * (m >> 2) + col][m & 3];
      return s;
    };
    if (m < a.m) {
      if constexpr (SWIGLU) {
        const int f = blockIdx.x * 8 + nn;
        if (nn < 8 && f < a.n_out) {
          st_agent(a.y + (int64_t)m * a.ldy + f, gated_act(total(nn), total(nn + 8), a.act_lut));
        }
      } else {
        const int o = blockIdx.x * 16 + nn;
        if (o < a.n_out) st_agent(a.y + (int64_t)m * a.ldy + o, f32_to_bf16(total(nn)));
      }
    }
  }
  stores_done();
}


// ---------------------------------------------------------------------------
// The same GEMM with the GEMV's 16-byte weight loads.  Lane l = 16 j + n of
// a wave reads block pair 4t + j of weight row n (two 16-byte loads and one
// 4-byte load, as the GEMV); a 4x4 transpose across the lanes n + 16 j
// (v_permlane16_swap / v_permlane32_swap) then gives lane (n, g) the k-group
// g of all 8 blocks of the tile: with the k-order of a block chosen as
// group g = elements 8g..8g+7 (low nibbles of qs[8g..8g+7] for g < 2, high
// nibbles of qs[8(g-2)..] for g >= 2), each group needs one 8-byte half of
// a block's qs and the activations of a group are 16 contiguous bytes of x.
// One v_mfma_f32_16x16x32_bf16 per block (A = activation row n, B = weight
// row n as bf16 128 + nibble) plus one against the constant -136, scaled by
// the block's fp16 d in fp32 (the scales travel through the same transpose).
// The waves of a workgroup take the tiles t = wave, wave + ks, ...
// ---------------------------------------------------------------------------

// 4x4 transpose across the four 16-lane rows: on entry row j of r_g holds
// X[j][g]; on exit row g of r_k holds X[k][g].  v_permlane16_swap(a, b)
// swaps the odd rows of a with the even rows of b; v_permlane32_swap(a, b)
// swaps rows 2-3 of a with rows 0-1 of b.
__device__ __forceinline__ void transpose_rows4(uint32_t& r0, uint32_t& r1, uint32_t& r2,
                                                uint32_t& r3) {
  const auto a = __builtin_amdgcn_permlane16_swap(r0, r1, false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(r2, r3, false, false);
  const auto c = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
  const auto d = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
  r0 = c[0];
  r2 = c[1];
  r1 = d[0];
  r3 = d[1];
}

// WS > 0 (m <= 2 WS <= 8): a wave copies its tile's activations -- m rows x
// 512 bytes, WS 16-byte loads per lane -- into a private LDS slice and reads
// the MFMA A operands from there (8 loads per tile straight from global
// memory cost 8 vector-memory instructions per tile whatever m is).  Chunk
// c of row r sits at 16 (r * 32 + (c ^ (r & 7))) bytes of the slice, so the
// rows of one operand read fall in different banks.
// KEYS (plain outputs): besides y, keys[row][blockIdx.x] is the greedy-argmax
// key of the workgroup's 16 outputs of each row (bf16_order_key), which the
// step-advance kernel reduces; the separate argmax launch is not needed.
template <bool SWIGLU, int WS, bool KEYS = false>
__global__ __launch_bounds__(1024) void q4_0_gemm_tile_kernel(
    const uint8_t* w_, const uint16_t* x_, int npairs, int n_out, int64_t up_offset_rows, int ks,
    int m, int64_t ldx, uint16_t* y, int64_t ldy, uint64_t* keys, const uint16_t* act_lut) {
  static_assert(!(SWIGLU && KEYS), "argmax keys are for plain outputs");
  __shared__ f32x4 red[16][64];
  extern __shared__ u32x4 xsl[];  // WS > 0: [ks][8 rows x 32 chunks]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, j = lane >> 4;  // j is also the lane's k-group after the transpose
  int wrow;
  if constexpr (SWIGLU) {
    const int f = min((int)blockIdx.x * 8 + (n & 7), n_out - 1);
    wrow = f + (n >= 8 ? (int)up_offset_rows : 0);
  } else {
    wrow = min((int)blockIdx.x * 16 + n, n_out - 1);
  }
  const uint8_t* wr = w_ + (int64_t)wrow * npairs * 36;
  const uint16_t* xr = x_ + (int64_t)min(n, m - 1) * ldx;  // rows >= m only feed unused C rows
  const int ntiles = (npairs + 3) >> 2;
  const uint32_t hshift = (uint32_t)(j >> 1) * 4u;  // high nibbles for k-groups 2 and 3
  bf16x8 bneg;
  {
    const uint32_t c[4] = {kNeg136, kNeg136, kNeg136, kNeg136};
    bneg = __builtin_bit_cast(bf16x8, c);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = zero;
  for (int t = wave; t < ntiles; t += ks) {
    // this lane's pair (clamped; a pair past the row end gets scale 0)
    const int pj = 4 * t + j;
    const uint32_t* pw = reinterpret_cast<const uint32_t*>(wr + 36 * min(pj, npairs - 1));
    const u32x4 pa = *reinterpret_cast<const u32x4_a4*>(pw);
    const u32x4 pb = *reinterpret_cast<const u32x4_a4*>(pw + 4);
    const uint32_t p8 = pw[8];
    // the activations of the tile's 8 blocks for this lane's row and k-group
    u32x4 xa[8];
    if constexpr (WS > 0) {
      u32x4* sl = xsl + wave * 256;
      u32x4 sv[WS];
#pragma unroll
      for (int i = 0; i < WS; ++i) {  // chunk c: row c >> 5, pair (c & 31) >> 3, 8 elements c & 7
        const int c = i * 64 + lane;
        const int pp = min(4 * t + ((c & 31) >> 3), npairs - 1);
        sv[i] = *reinterpret_cast<const u32x4*>(x_ + (int64_t)min(c >> 5, m - 1) * ldx + pp * 64 +
                                                (c & 7) * 8);
      }
#pragma unroll
      for (int i = 0; i < WS; ++i) {
        const int c = i * 64 + lane, r = c >> 5;
        sl[r * 32 + ((c & 31) ^ (r & 7))] = sv[i];
      }
      // the slice is private to this wave: its LDS operations complete in
      // order, so only the compiler has to be kept from reordering
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int xrow = min(n, m - 1);
#pragma unroll
      for (int b = 0; b < 8; ++b)
        xa[b] = sl[xrow * 32 + ((((b >> 1) * 8 + (b & 1) * 4 + j)) ^ (xrow & 7))];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    } else {
#pragma unroll
      for (int b = 0; b < 8; ++b) {
        const int pp = min(4 * t + (b >> 1), npairs - 1);
        xa[b] = *reinterpret_cast<const u32x4*>(xr + pp * 64 + (b & 1) * 32 + 8 * j);
      }
    }
    // qs dwords of the even block (bytes 2..17 of the pair) and the odd one
    // (bytes 20..35), and the two scales packed (d_even | d_odd << 16)
    const uint32_t qe0 = perm_b32(pa.y, pa.x, 0x05040302u);
    const uint32_t qe1 = perm_b32(pa.z, pa.y, 0x05040302u);
    const uint32_t qe2 = perm_b32(pa.w, pa.z, 0x05040302u);
    const uint32_t qe3 = perm_b32(pb.x, pa.w, 0x05040302u);
    const uint32_t dd = pj < npairs ? perm_b32(pb.x, pa.x, 0x07060100u) : 0u;
    // k-group g takes the 8-byte half g & 1 of each block's qs
    uint32_t ea0 = qe0, ea1 = qe2, ea2 = qe0, ea3 = qe2;
    uint32_t eb0 = qe1, eb1 = qe3, eb2 = qe1, eb3 = qe3;
    uint32_t oa0 = pb.y, oa1 = pb.w, oa2 = pb.y, oa3 = pb.w;
    uint32_t ob0 = pb.z, ob1 = p8, ob2 = pb.z, ob3 = p8;
    uint32_t d0 = dd, d1 = dd, d2 = dd, d3 = dd;
    transpose_rows4(ea0, ea1, ea2, ea3);
    transpose_rows4(eb0, eb1, eb2, eb3);
    transpose_rows4(oa0, oa1, oa2, oa3);
    transpose_rows4(ob0, ob1, ob2, ob3);
    transpose_rows4(d0, d1, d2, d3);
    const uint32_t qa[8] = {ea0, oa0, ea1, oa1, ea2, oa2, ea3, oa3};  // block b = 2k + odd
    const uint32_t qb[8] = {eb0, ob0, eb1, ob1, eb2, ob2, eb3, ob3};
    const uint32_t dk[4] = {d0, d1, d2, d3};
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const uint32_t lo = (qa[b] >> hshift) & kNibG;
      const uint32_t hi = (qb[b] >> hshift) & kNibG;
      const uint32_t bw[4] = {perm_b32(kMagicG, lo, kSel01G), perm_b32(kMagicG, lo, kSel23G),
                              perm_b32(kMagicG, hi, kSel01G), perm_b32(kMagicG, hi, kSel23G)};
      const bf16x8 A = __builtin_bit_cast(bf16x8, xa[b]);
      f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, bw), zero,
                                                        0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, bneg, c, 0, 0, 0);
      const float d = f16_bits_to_f32((b & 1) ? (dk[b >> 1] >> 16) : (dk[b >> 1] & 0xffffu));
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, c[r], acc[r]);
    }
  }
  // C layout: lane l holds rows 4 (l >> 4) + r of column l & 15.
  red[wave][lane] = acc;
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 64 * ks) {  // 16 rows x 16 columns
    const int mr = e >> 4, nn = e & 15;
    auto total = [&](int col) {
      float s = 0.f;
      for (int w = 0; w < ks; ++w) s += red[w][16 * (mr >> 2) + col][mr & 3];
      return s;
    };
    if (mr < m) {
      if constexpr (SWIGLU) {
        const int f = blockIdx.x * 8 + nn;
        if (nn < 8 && f < n_out) {
          st_agent(y + (int64_t)mr * ldy + f, gated_act(total(nn), total(nn + 8), act_lut));
        }
      } else {
        const int o = blockIdx.x * 16 + nn;
        if (o < n_out) st_agent(y + (int64_t)mr * ldy + o, f32_to_bf16(total(nn)));
      }
    }
    if constexpr (KEYS && !SWIGLU) {
      // the 16 outputs of row mr sit in lanes 16 q .. 16 q + 15 of this wave
      const int o = blockIdx.x * 16 + nn;
      uint64_t key = 0;
      if (mr < m && o < n_out)
        key = ((uint64_t)bf16_order_key(f32_to_bf16(total(nn))) << 32) |
              (uint64_t)(0xffffffffu - (uint32_t)o);
#pragma unroll
      for (int s = 1; s < 16; s <<= 1) {
        const uint64_t other =
            ((uint64_t)(uint32_t)__shfl_xor((int)(key >> 32), s, 64) << 32) |
            (uint32_t)__shfl_xor((int)(uint32_t)key, s, 64);
        key = other > key ? other : key;
      }
      // one key per row and 16-column group (the grid is ceil(n_out / 16) workgroups)
      if (nn == 0 && mr < m) st_agent(keys + (int64_t)mr * ((n_out + 15) / 16) + blockIdx.x, key);
    }
  }
  stores_done();
}

template <bool SWIGLU, bool KEYS = false>
hipError_t launch_gemm_tile(hipStream_t s, const void* x, const void* w, void* y, int64_t m,
                            int64_t n_out, int64_t k, int64_t up_offset_rows,
                            uint64_t* keys = nullptr, const uint16_t* act_lut = nullptr) {
  const int npairs = (int)(k / 64);
  const int ntiles = (npairs + 3) / 4;
  const int grid = SWIGLU ? (int)((n_out + 7) / 8) : (int)((n_out + 15) / 16);
  // Waves per workgroup (each takes every ks-th K tile), measured at 8 rows:
  // many workgroups want small ones, more of them resident per CU (head
  // 151936x2560: 4 waves 69.3 µs, 10 waves 89.7; gate/up 19456x2560: 5 waves
  // 12.4, 10 waves 14.1), few workgroups up to 10 (down 2560x9728, 38 tiles:
  // 10 waves 8.4, 16 waves 9.3; QKV and o_proj within 1 % from 10 to 16).
  int ks = grid >= 4096 ? 4 : grid >= 1024 ? (ntiles + 1) / 2 : 10;
  if (const char* e = tuning_env("SMX_GEMM_KS")) {  // tuning sweeps
    const int v = atoi(e);
    if (v >= 1 && v <= 16) ks = v;
  }
  ks = ks < 1 ? 1 : ks > 16 ? 16 : ks;
  ks = ks < ntiles ? ks : ntiles;
  int ws = m <= 2 ? 1 : m <= 4 ? 2 : m <= 8 ? 4 : 0;
  if (const char* e = tuning_env("SMX_GEMM_WS")) ws = atoi(e) ? ws : 0;  // tuning sweeps
  const size_t lds = ws ? (size_t)ks * 256 * 16 : 0;
#define SMX_GEMM_LAUNCH(W)                                                                      \
  SMX_LAUNCH((q4_0_gemm_tile_kernel<SWIGLU, W, KEYS>), dim3(grid), dim3(64 * ks), lds,  \
                     s, (const uint8_t*)w, (const uint16_t*)x, npairs, (int)n_out,                \
                     up_offset_rows, ks, (int)m, k, (uint16_t*)y, n_out, keys, act_lut)
  if (ws == 1) SMX_GEMM_LAUNCH(1);
  else if (ws == 2) SMX_GEMM_LAUNCH(2);
  else if (ws == 4) SMX_GEMM_LAUNCH(4);
  else SMX_GEMM_LAUNCH(0);
#undef SMX_GEMM_LAUNCH
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Packed layout (smx_q4_0_repack): the tile kernel's MFMA B operands stored
// lane by lane, so a wave reads a 16-row x 256-k chunk with three 16-byte
// loads and no cross-lane transposes.  Chunk c of row group G is 2304 bytes
// at (G * nchunks + c) * 2304:
//   [0, 1024)     lane l (row n = l & 15, k-group g = l >> 4): 16 bytes, word
//                 i = block i of the chunk, whose byte b holds the codes of the
//                 block's elements 8 g + b (low nibble) and 8 g + 4 + b (high)
//   [1024, 2048)  the same for blocks 4..7
//   [2048, 2304)  row n's 8 fp16 scales at 2048 + 16 n
// Row n of group G is weight row 16 G + n (plain), or, gated, gate row
// 8 G + n for n < 8 and up row d + 8 G + n - 8 otherwise; rows past the end
// repeat the last row (their outputs are never stored).  The bytes are the
// GGUF blocks' own codes and scales, moved: the repack is lossless.
// ---------------------------------------------------------------------------
constexpr int kChunkBytes = 2304;

// One thread per (group, chunk, lane); row-major reads of the GGUF blocks.
__global__ __launch_bounds__(256) void q4_0_repack_kernel(const uint8_t* __restrict__ w,
                                                          uint8_t* __restrict__ out, int n_out,
                                                          int nblocks, int gated, int ngroups) {
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nchunks = nblocks / 8;
  if (tid >= (int64_t)ngroups * nchunks * 64) return;
  const int l = (int)(tid & 63);
  const int64_t gc = tid >> 6;
  const int c = (int)(gc % nchunks), G = (int)(gc / nchunks);
  const int n = l & 15, g = l >> 4;
  int64_t row;
  if (gated) row = min(G * 8 + (n & 7), n_out - 1) + (n >= 8 ? (int64_t)n_out : 0);
  else row = min(G * 16 + n, n_out - 1);
  const uint8_t* rw = w + row * (int64_t)nblocks * 18;
  uint8_t* base = out + gc * kChunkBytes;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    uint32_t words[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* qs = rw + (c * 8 + part * 4 + i) * 18 + 2;
      // element e of a block: low nibble of qs[e] (e < 16), else high nibble of qs[e - 16]
      auto code = [&](int e) -> uint32_t { return e < 16 ? (qs[e] & 15u) : (qs[e - 16] >> 4); };
      uint32_t wd = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) wd |= (code(8 * g + b) | (code(8 * g + 4 + b) << 4)) << (8 * b);
      words[i] = wd;
    }
    st_agent(reinterpret_cast<u32x4*>(base + part * 1024 + 16 * l),
             u32x4{words[0], words[1], words[2], words[3]});
  }
  if (g == 0) {
    uint32_t sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint8_t* b0 = rw + (c * 8 + 2 * i) * 18;
      const uint8_t* b1 = b0 + 18;
      sc[i] = (uint32_t)b0[0] | ((uint32_t)b0[1] << 8) | ((uint32_t)b1[0] << 16) | ((uint32_t)b1[1] << 24);
    }
    st_agent(reinterpret_cast<u32x4*>(base + 2048 + 16 * n), u32x4{sc[0], sc[1], sc[2], sc[3]});
  }
  stores_done();
}

// The tile kernel's arithmetic over the packed layout: per 256-k chunk a lane
// loads its 8 blocks' B words and its row's 8 scales directly; the
// activations are staged through the wave's LDS slice as in the tile kernel
// (WS 16-byte loads per lane, m <= 2 WS rows).  Per block: MFMA(A, 128 +
// code), MFMA(A, -136) and the fp32 scale; the waves of a workgroup (ks <=
// 10) take the chunks t = wave, wave + ks, ... and are summed in wave order.
template <bool SWIGLU, int WS, bool KEYS = false>
__global__ __launch_bounds__(640) void q4_0_gemm_packed_kernel(
    const uint8_t* wp, const uint16_t* x_, int nchunks, int n_out, int ks, int m, int64_t ldx,
    uint16_t* y, int64_t ldy, uint64_t* keys, const uint16_t* act_lut) {
  static_assert(!(SWIGLU && KEYS), "argmax keys are for plain outputs");
  __shared__ f32x4 red[10][64];
  extern __shared__ u32x4 xsl[];  // [ks][2 WS rows x 32 chunks]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, j = lane >> 4;
  const uint8_t* gbase = wp + (int64_t)blockIdx.x * nchunks * kChunkBytes;
  bf16x8 bneg;
  {
    const uint32_t c[4] = {kNeg136, kNeg136, kNeg136, kNeg136};
    bneg = __builtin_bit_cast(bf16x8, c);
  }
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = zero;
  const int xrow = min(n, m - 1);  // rows >= m only feed unused C rows
  // chunk t + ks's weights and activations are loaded while chunk t is
  // computed (the next chunk's loads are issued once this chunk's registers
  // have been consumed)
  u32x4 wa, wb, sc, sv[WS];
  auto load = [&](int t) {
    const uint8_t* cb = gbase + (int64_t)t * kChunkBytes;
    wa = *reinterpret_cast<const u32x4*>(cb + 16 * lane);
    wb = *reinterpret_cast<const u32x4*>(cb + 1024 + 16 * lane);
    sc = *reinterpret_cast<const u32x4*>(cb + 2048 + 16 * n);
#pragma unroll
    for (int i = 0; i < WS; ++i) {  // piece q: row q >> 5, 16 bytes (q & 31) of the chunk
      const int q = i * 64 + lane;
      sv[i] = *reinterpret_cast<const u32x4*>(x_ + (int64_t)min(q >> 5, m - 1) * ldx + t * 256 +
                                              (q & 31) * 8);
    }
  };
  if (wave < nchunks) load(wave);
  for (int t = wave; t < nchunks; t += ks) {
    u32x4 xa[8];
    {
      u32x4* sl = xsl + wave * (WS * 64);
#pragma unroll
      for (int i = 0; i < WS; ++i) {
        const int q = i * 64 + lane, r = q >> 5;
        sl[r * 32 + ((q & 31) ^ (r & 7))] = sv[i];
      }
      // the slice is private to this wave (see the tile kernel)
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int b = 0; b < 8; ++b) xa[b] = sl[xrow * 32 + ((4 * b + j) ^ (xrow & 7))];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    const uint32_t wd[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
    const uint32_t sd[4] = {sc.x, sc.y, sc.z, sc.w};
    if (t + ks < nchunks) load(t + ks);
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const bf16x8 A = __builtin_bit_cast(bf16x8, xa[b]);
      f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, dequant_word(wd[b]), zero, 0, 0, 0);
      c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, bneg, c, 0, 0, 0);
      const float d = f16_bits_to_f32((b & 1) ? (sd[b >> 1] >> 16) : (sd[b >> 1] & 0xffffu));
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = fmaf(d, c[r], acc[r]);
    }
  }
  // C layout: lane l holds rows 4 (l >> 4) + r of column l & 15.
  red[wave][lane] = acc;
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += 64 * ks) {  // 16 rows x 16 columns
    const int mr = e >> 4, nn = e & 15;
    auto total = [&](int col) {
      float s = 0.f;
      for (int w = 0; w < ks; ++w) s += red[w][16 * (mr >> 2) + col][mr & 3];
      return s;
    };
    if (mr < m) {
      if constexpr (SWIGLU) {
        const int f = blockIdx.x * 8 + nn;
        if (nn < 8 && f < n_out) {
          st_agent(y + (int64_t)mr * ldy + f, gated_act(total(nn), total(nn + 8), act_lut));
        }
      } else {
        const int o = blockIdx.x * 16 + nn;
        if (o < n_out) st_agent(y + (int64_t)mr * ldy + o, f32_to_bf16(total(nn)));
      }
    }
    if constexpr (KEYS && !SWIGLU) {
      const int o = blockIdx.x * 16 + nn;
      uint64_t key = 0;
      if (mr < m && o < n_out)
        key = ((uint64_t)bf16_order_key(f32_to_bf16(total(nn))) << 32) |
              (uint64_t)(0xffffffffu - (uint32_t)o);
#pragma unroll
      for (int s = 1; s < 16; s <<= 1) {
        const uint64_t other =
            ((uint64_t)(uint32_t)__shfl_xor((int)(key >> 32), s, 64) << 32) |
            (uint32_t)__shfl_xor((int)(uint32_t)key, s, 64);
        key = other > key ? other : key;
      }
      if (nn == 0 && mr < m) st_agent(keys + (int64_t)mr * ((n_out + 15) / 16) + blockIdx.x, key);
    }
  }
  stores_done();
}

inline int64_t packed_groups(int64_t n, bool gated) { return gated ? (n + 7) / 8 : (n + 15) / 16; }

template <bool SWIGLU, bool KEYS = false>
hipError_t launch_gemm_packed(hipStream_t s, const void* x, const void* wp, void* y, int64_t m,
                              int64_t n_out, int64_t k, uint64_t* keys = nullptr,
                              const uint16_t* act_lut = nullptr) {
  const int nchunks = (int)(k / 256);
  const int grid = (int)packed_groups(n_out, SWIGLU);
  // Waves per workgroup, measured at 8 rows (µs, ks): gate/up 19456x2560
  // 9.39 (2), 10.22 (3); head 151936x2560 57.3 (2), 58.1 (3); QKV 6144x2560
  // 5.25 (6), 5.31 (4), 6.37 (10); o_proj 2560x4096 4.46 (8), 4.50 (10),
  // 5.25 (4); down 2560x9728 7.41 (10), 7.51 (8), 9.48 (4).
  int ks = grid >= 1024 ? 2 : grid >= 256 ? 5 : 10;
  if (const char* e = tuning_env("SMX_PACKED_KS")) {  // tuning sweeps
    const int v = atoi(e);
    if (v >= 1 && v <= 10) ks = v;
  }
  ks = ks < nchunks ? ks : nchunks;
  const int ws = m <= 2 ? 1 : m <= 4 ? 2 : m <= 8 ? 4 : 8;
  const size_t lds = (size_t)ks * ws * 64 * 16;
#define SMX_PACKED_LAUNCH(W)                                                                    \
  SMX_LAUNCH((q4_0_gemm_packed_kernel<SWIGLU, W, KEYS>), dim3(grid), dim3(64 * ks), lds, s,     \
             (const uint8_t*)wp, (const uint16_t*)x, nchunks, (int)n_out, ks, (int)m, k,         \
             (uint16_t*)y, n_out, keys, act_lut)
  if (ws == 1) SMX_PACKED_LAUNCH(1);
  else if (ws == 2) SMX_PACKED_LAUNCH(2);
  else if (ws == 4) SMX_PACKED_LAUNCH(4);
  else SMX_PACKED_LAUNCH(8);
#undef SMX_PACKED_LAUNCH
  return hipGetLastError();
}
}  // namespace
}  // namespace smx

#include "smx_abi_util.h"


#define SMX_GEMM_CHECKS(N)                                                                      \
  SMX_REQUIRE(x && w && y, "null pointer argument");                                            \
  SMX_REQUIRE(m >= 1 && m <= 16, "m must be in [1, 16]");                                       \
  SMX_REQUIRE((N) >= 1 && (N) <= (1ll << 30), "bad output size");                               \
  SMX_REQUIRE(k >= 64 && k % 64 == 0 && k <= (1 << 20), "k must be a positive multiple of 64"); \
  SMX_REQUIRE((uintptr_t)x % 8 == 0 && (uintptr_t)w % 4 == 0 && (uintptr_t)y % 2 == 0,          \
              "x must be 8-byte aligned, w 4-byte aligned")

extern "C" int smx_q4_0_gemm(void* stream, const void* x, const void* w, void* y, int64_t m,
                             int64_t n, int64_t k) {
  SMX_GEMM_CHECKS(n);
  if ((uintptr_t)x % 16 == 0)
    return (int)smx::launch_gemm_tile<false>((hipStream_t)stream, x, w, y, m, n, k, 0);
  smx::GemmArgs a{(const uint16_t*)x, (const uint8_t*)w, (uint16_t*)y, (int)m, (int)n,
                  (int)(k / 64), k, n, 0};
  SMX_LAUNCH(smx::q4_0_gemm_kernel<false>, dim3((unsigned)((n + 15) / 16)), dim3(512), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

static int gemm_gated(void* stream, const void* x, const void* w, const void* lut, void* y,
                      int64_t m, int64_t d, int64_t k) {
  const uint16_t* act_lut = (const uint16_t*)lut;
  if ((uintptr_t)x % 16 == 0)
    return (int)smx::launch_gemm_tile<true>((hipStream_t)stream, x, w, y, m, d, k, d, nullptr,
                                            act_lut);
  smx::GemmArgs a{(const uint16_t*)x, (const uint8_t*)w, (uint16_t*)y, (int)m, (int)d,
                  (int)(k / 64), k, d, d, act_lut};
  SMX_LAUNCH(smx::q4_0_gemm_kernel<true>, dim3((unsigned)((d + 7) / 8)), dim3(512), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

extern "C" int smx_q4_0_gemm_swiglu(void* stream, const void* x, const void* w, void* y,
                                    int64_t m, int64_t d, int64_t k) {
  SMX_GEMM_CHECKS(d);
  return gemm_gated(stream, x, w, nullptr, y, m, d, k);
}

extern "C" int smx_q4_0_gemm_gelu(void* stream, const void* x, const void* w, const void* lut,
                                  void* y, int64_t m, int64_t d, int64_t k) {
  SMX_GEMM_CHECKS(d);
  SMX_REQUIRE(lut && (uintptr_t)lut % 2 == 0, "lut must be non-null and 2-byte aligned");
  return gemm_gated(stream, x, w, lut, y, m, d, k);
}

extern "C" int64_t smx_q4_0_gemm_keys_per_row(int64_t n) { return (n + 15) / 16; }

extern "C" int smx_q4_0_gemm_argmax(void* stream, const void* x, const void* w, void* y,
                                    uint64_t* keys, int64_t m, int64_t n, int64_t k) {
  SMX_GEMM_CHECKS(n);
  SMX_REQUIRE(keys && (uintptr_t)keys % 8 == 0, "keys must be non-null and 8-byte aligned");
  SMX_REQUIRE((uintptr_t)x % 16 == 0, "x must be 16-byte aligned");
  return (int)smx::launch_gemm_tile<false, true>((hipStream_t)stream, x, w, y, m, n, k, 0, keys);
}

// ---------------------------------------------------------------------------
// The packed layout's entry points.

extern "C" int64_t smx_q4_0_packed_bytes(int64_t n, int64_t k, int gated) {
  if (n < 1 || n > (1ll << 30) || k < 256 || k % 256 != 0 || k > (1 << 20)) return -1;
  return smx::packed_groups(n, gated != 0) * (k / 256) * smx::kChunkBytes;
}

extern "C" int smx_q4_0_repack(void* stream, const void* w, void* wp, int64_t n, int64_t k,
                               int gated) {
  SMX_REQUIRE(w && wp, "null pointer argument");
  SMX_REQUIRE(smx_q4_0_packed_bytes(n, k, gated) > 0,
              "n must be in [1, 2^30] and k a positive multiple of 256 (at most 2^20)");
  SMX_REQUIRE((uintptr_t)wp % 16 == 0, "wp must be 16-byte aligned");
  const int64_t groups = smx::packed_groups(n, gated != 0);
  const int64_t threads = groups * (k / 256) * 64;
  SMX_REQUIRE((threads + 255) / 256 <= 0x7fffffff, "matrix too large for one repack launch");
  SMX_LAUNCH(smx::q4_0_repack_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
             (hipStream_t)stream, (const uint8_t*)w, (uint8_t*)wp, (int)n, (int)(k / 32),
             gated ? 1 : 0, (int)groups);
  return (int)hipGetLastError();
}

#define SMX_PACKED_CHECKS(N)                                                                    \
  SMX_REQUIRE(x && wp && y, "null pointer argument");                                           \
  SMX_REQUIRE(m >= 1 && m <= 16, "m must be in [1, 16]");                                       \
  SMX_REQUIRE((N) >= 1 && (N) <= (1ll << 30), "bad output size");                               \
  SMX_REQUIRE(k >= 256 && k % 256 == 0 && k <= (1 << 20),                                       \
              "k must be a positive multiple of 256");                                          \
  SMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)wp % 16 == 0 && (uintptr_t)y % 2 == 0,       \
              "x and wp must be 16-byte aligned")

extern "C" int smx_q4_0_gemm_packed(void* stream, const void* x, const void* wp, void* y,
                                    int64_t m, int64_t n, int64_t k) {
  SMX_PACKED_CHECKS(n);
  return (int)smx::launch_gemm_packed<false>((hipStream_t)stream, x, wp, y, m, n, k);
}

extern "C" int smx_q4_0_gemm_packed_swiglu(void* stream, const void* x, const void* wp, void* y,
                                           int64_t m, int64_t d, int64_t k) {
  SMX_PACKED_CHECKS(d);
  return (int)smx::launch_gemm_packed<true>((hipStream_t)stream, x, wp, y, m, d, k);
}

extern "C" int smx_q4_0_gemm_packed_gelu(void* stream, const void* x, const void* wp,
                                         const void* lut, void* y, int64_t m, int64_t d,
                                         int64_t k) {
  SMX_PACKED_CHECKS(d);
  SMX_REQUIRE(lut && (uintptr_t)lut % 2 == 0, "lut must be non-null and 2-byte aligned");
  return (int)smx::launch_gemm_packed<true>((hipStream_t)stream, x, wp, y, m, d, k, nullptr,
                                            (const uint16_t*)lut);
}

extern "C" int smx_q4_0_gemm_packed_argmax(void* stream, const void* x, const void* wp, void* y,
                                           uint64_t* keys, int64_t m, int64_t n, int64_t k) {
  SMX_PACKED_CHECKS(n);
  SMX_REQUIRE(keys && (uintptr_t)keys % 8 == 0, "keys must be non-null and 8-byte aligned");
  return (int)smx::launch_gemm_packed<false, true>((hipStream_t)stream, x, wp, y, m, n, k, keys);
}
