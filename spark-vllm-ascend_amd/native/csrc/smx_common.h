// Device helpers shared by the gfx950 kernels of the Q4_0 decode path.
#pragma once

#include <stdlib.h>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../../include/smx.h"

namespace smx {

// Launch-shape overrides for tuning sweeps: read only when SMX_TUNE is set
// in the environment (looked up once per process), so a production launch
// never calls getenv.
inline const char* tuning_env(const char* name) {
  static const bool on = getenv("SMX_TUNE") != nullptr;
  return on ? getenv(name) : nullptr;
}


typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Stores of values that another kernel reads.  They are agent-scope (sc1)
// stores: written through this XCD's L2 to the device's coherence point,
// where a kernel on any XCD that starts after this one has ended reads them,
// so the boundary between the two kernels needs no L2 write-back (the
// step runner's acquire-only fence mode relies on it).  Every kernel calls
// stores_done() after its last such store: its waves end only once the
// stores have completed.
template <typename T>
__device__ __forceinline__ void st_agent(T* p, T v) {
  static_assert(sizeof(T) == 1 || sizeof(T) == 2 || sizeof(T) == 4 || sizeof(T) == 8,
                "8- to 64-bit stores");
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  st_agent(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
__device__ __forceinline__ void st_agent(u32x2* p, u32x2 v) {
  st_agent(reinterpret_cast<uint64_t*>(p), (uint64_t)v.x | ((uint64_t)v.y << 32));
}
__device__ __forceinline__ void st_agent(u32x4* p, u32x4 v) {  // two 64-bit stores
  uint64_t* q = reinterpret_cast<uint64_t*>(p);
  st_agent(q, (uint64_t)v.x | ((uint64_t)v.y << 32));
  st_agent(q + 1, (uint64_t)v.z | ((uint64_t)v.w << 32));
}
__device__ __forceinline__ void stores_done() { __builtin_amdgcn_s_waitcnt(0); }

// Unaligned-to-16 (but 4-byte aligned) vector types for the Q4_0 stream:
// GGUF blocks are 18 bytes, so a block pair starts on a 4-byte boundary only.
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h16) {
  return __uint_as_float(h16 << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// float -> bf16 bits, round to nearest even (NaN stays NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ float round_bf16(float f) {
  return bf16_bits_to_f32(f32_to_bf16(f));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h16) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

// erf-GELU of a bf16 gate through the table of the reference's gate/up
// activation (src/spark_vllm_ascend/kernels/linear.py:540-577, table built at
// src/spark_vllm_ascend/integration/model.py:13-16): lut[0, 2048) holds
// gelu(g) for the bf16 bit patterns 0x3b00..0x42ff (2^-9 <= g < 128) and
// lut[2048, 4096) for 0xbb00..0xc2ff (their negatives).  Outside the table:
// |g| < 2^-9 gives g / 2, g >= 128 gives g (+inf stays +inf), g <= -128
// gives -0, NaN and -inf give the NaN 0x7fff.
constexpr int kGeluLutEntries = 4096;
__device__ __forceinline__ uint16_t gelu_lut(uint32_t g, const uint16_t* lut) {
  const uint32_t ab = g & 0x7fffu;
  if (ab > 0x7f80u || g == 0xff80u) return 0x7fffu;
  if (ab >= 0x4300u) return g < 0x8000u ? (uint16_t)g : (uint16_t)0x8000u;
  if (ab < 0x3b00u) return f32_to_bf16(0.5f * bf16_bits_to_f32(g));
  return lut[((ab - 0x3b00u) & 2047u) | ((g >> 4) & 2048u)];
}

// The gated-MLP activation of the GEMV/GEMM epilogues, on the fp32 sums of a
// gate row and its up row, each first rounded to bf16 (the GEMV output):
// silu(g) * u in fp32 when lut is null (SwiGLU), else gelu_lut(g) * u.
__device__ __forceinline__ uint16_t gated_act(float gate_sum, float up_sum, const uint16_t* lut) {
  const uint16_t gbits = f32_to_bf16(gate_sum);
  const float gb = bf16_bits_to_f32(gbits);
  const float ub = round_bf16(up_sum);
  if (lut) return f32_to_bf16(bf16_bits_to_f32(gelu_lut(gbits, lut)) * ub);
  return f32_to_bf16(gb / (1.0f + expf(-gb)) * ub);
}

// Order-preserving 16-bit key of a bf16 value (NaN above +inf).  Greedy
// argmax keys are (key << 32) | (0xffffffff - index): the largest key is the
// largest value, the lowest index among equal values.
__device__ __forceinline__ uint32_t bf16_order_key(uint16_t b) {
  if ((b & 0x7f80u) == 0x7f80u && (b & 0x7fu)) return 0xffffu;  // NaN
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}

// acc + a.lo*b.lo + a.hi*b.hi, both operands packed bf16 pairs (v_dot2c_f32_bf16).
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                         __builtin_bit_cast(bf16x2, b), acc, false);
}

// v_perm_b32: byte i of the result is byte sel[i] of the 8-byte value {hi, lo}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

// DPP lane moves inside one 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// DPP control words (GCN/CDNA encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// Sum over each aligned group of 8 lanes; every lane of the group gets it.
__device__ __forceinline__ float sum8(float v) {
  v += dpp_f32<DPP_QUAD_XOR1>(v);
  v += dpp_f32<DPP_QUAD_XOR2>(v);
  v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
  return v;
}
// Sum over each aligned group of 4 lanes.
__device__ __forceinline__ float sum4(float v) {
  v += dpp_f32<DPP_QUAD_XOR1>(v);
  v += dpp_f32<DPP_QUAD_XOR2>(v);
  return v;
}

// This lane's value and that of lane ^ MASK (MASK 16 or 32), in an order that
// differs between the two lanes: v_permlane16_swap_b32 / v_permlane32_swap_b32
// of a register with itself exchange its odd 16-lane rows (odd 32-lane
// halves) with the even ones of the copy, so each lane ends with {own,
// partner}.  Plain VALU operations, where __shfl_xor goes through the LDS
// crossbar (ds_bpermute, an LDS round trip).  All 64 lanes must be active.
// Sums and maxima over the pair are commutative, so every lane of a pair
// gets the same bits.
template <int MASK>
__device__ __forceinline__ void lane_pair(float v, float& a, float& b) {
  static_assert(MASK == 16 || MASK == 32, "row swaps of 16 or 32 lanes");
  const uint32_t u = __float_as_uint(v);
  if constexpr (MASK == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
  }
}
template <int MASK>
__device__ __forceinline__ float xor_sum(float v) {
  float a, b;
  lane_pair<MASK>(v, a, b);
  return a + b;
}
template <int MASK>
__device__ __forceinline__ float xor_max(float v) {
  float a, b;
  lane_pair<MASK>(v, a, b);
  return fmaxf(a, b);
}

// Full-wave reductions.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<DPP_QUAD_XOR1>(v);
  v += dpp_f32<DPP_QUAD_XOR2>(v);
  v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
  v += dpp_f32<DPP_ROW_MIRROR>(v);
  v = xor_sum<16>(v);
  v = xor_sum<32>(v);
  return v;
}

}  // namespace smx
