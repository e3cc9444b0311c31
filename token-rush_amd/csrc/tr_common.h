// Shared device helpers for the gfx950 verify-path kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tr {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Error codes returned by every C-ABI entry point (0 = success). 1 and 2 keep the
// meaning the reference's Marlin launcher gives them (marlin_bf16.cu:627-669).
enum {
  TR_OK = 0,
  TR_ERR_SHAPE = 1,      // unsupported problem shape
  TR_ERR_CONFIG = 2,     // no kernel configuration for the requested tiling
  TR_ERR_ARG = 3,        // null pointer / bad enum / bad size
  TR_ERR_LAUNCH = 4,     // the HIP launch itself failed
};

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even (what torch's .to(bfloat16) does for finite values;
// NaN is kept a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// silu(g) * u in fp32, the MLP activation (tokenrush/fused.py:76). One definition for the fused
// GEMM epilogue and the stand-alone kernel, so the two paths agree bit for bit.
__device__ __forceinline__ float silu_mul_f32(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// A value the compiler must keep in a VGPR: lets v_and_or_b32 take (VGPR, SGPR, VGPR)
// operands, since a gfx9 VOP3 instruction reads at most one scalar/literal.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

}  // namespace tr
