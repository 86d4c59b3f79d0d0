// Q4_0 GEMM for a few activation rows (batched decode, M <= 16) on MFMA.
//
// Y[m][n] = sum_k X[m][k] * W[n][k] with W in GGUF Q4_0 blocks (fp16 d, 16
// bytes of nibbles, value d * (nibble - 8)), bf16 X and Y, fp32 accumulation
// -- the GEMV semantics of src/spark_vllm_ascend/kernels/linear.py:16-200 for
// several rows at once (the reference runs batch 1 only).
//
// One workgroup of 8 waves per 16 weight rows (one MFMA N-tile); the waves
// split the K dimension by block pairs and meet in LDS.  Per block, with
// v_mfma_f32_16x16x32_bf16 (A = X rows as the M side, B = W^T):
//  * lane l holds weight row n = l & 15 and k-slot group g = l >> 4: one
//    32-bit word of the block's nibbles, i.e. 8 weights, which v_perm_b32
//    turns into bf16 128 + nibble (the nibble spliced under the byte 0x43);
//  * C = A * B(128 + nibble) + A * B(-136) = sum_k x * (nibble - 8): the
//    offset is a second MFMA against a constant operand, so no per-block
//    activation sums are needed;
//  * the block result is scaled by the lane's row scale d in fp32.
// The K order inside an MFMA is a permutation shared by A and B: slot j of
// group g is the element of the word's byte j & 3, low nibble for j < 4 and
// high nibble (element + 16) otherwise.  Block pairs are 36 bytes, so the
// even block's nibbles start 2 bytes into a dword; its group-0 word is
// spliced from the pair's dwords 0 and 4 (elements 14, 15, 0, 1).
#include "smx_common.h"

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
          const float gb = round_bf16(total(nn));
          const float ub = round_bf16(total(nn + 8));
          a.y[(int64_t)m * a.ldy + f] = f32_to_bf16(gb / (1.0f + expf(-gb)) * ub);
        }
      } else {
        const int o = blockIdx.x * 16 + nn;
        if (o < a.n_out) a.y[(int64_t)m * a.ldy + o] = f32_to_bf16(total(nn));
      }
    }
  }
}

}  // namespace
}  // namespace smx

#include "smx_abi_util.h"

namespace smx {
// Multi-row streaming GEMV (q4_0_gemv.hip); hipErrorNotSupported for shapes
// it does not take (then the MFMA kernel above runs).
hipError_t q4_0_gemv_rows(hipStream_t s, const void* x, const void* w, void* y, int64_t m,
                          int64_t n_out, int64_t k, int64_t ldx, int64_t ldy, bool swiglu,
                          int64_t up_offset_rows);
}  // namespace smx

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
  {
    const hipError_t e = smx::q4_0_gemv_rows((hipStream_t)stream, x, w, y, m, n, k, k, n, false, 0);
    if (e != hipErrorNotSupported) return (int)e;
  }
  smx::GemmArgs a{(const uint16_t*)x, (const uint8_t*)w, (uint16_t*)y, (int)m, (int)n,
                  (int)(k / 64), k, n, 0};
  hipLaunchKernelGGL(smx::q4_0_gemm_kernel<false>, dim3((unsigned)((n + 15) / 16)), dim3(512), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}

extern "C" int smx_q4_0_gemm_swiglu(void* stream, const void* x, const void* w, void* y,
                                    int64_t m, int64_t d, int64_t k) {
  SMX_GEMM_CHECKS(d);
  {
    const hipError_t e = smx::q4_0_gemv_rows((hipStream_t)stream, x, w, y, m, d, k, k, d, true, d);
    if (e != hipErrorNotSupported) return (int)e;
  }
  smx::GemmArgs a{(const uint16_t*)x, (const uint8_t*)w, (uint16_t*)y, (int)m, (int)d,
                  (int)(k / 64), k, d, d};
  hipLaunchKernelGGL(smx::q4_0_gemm_kernel<true>, dim3((unsigned)((d + 7) / 8)), dim3(512), 0,
                     (hipStream_t)stream, a);
  return (int)hipGetLastError();
}
