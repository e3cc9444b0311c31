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
  TR_ERR_SCRATCH = 5,    // the call needs more than the fixed device scratch of a no-allocation entry point
};

// Ordering of the last-arriver handoffs (a workgroup publishes data, then bumps a counter; the
// last arriver reads everyone's data). The library's build publishes with agent-scope (sc1)
// stores, waits for them to complete, passes a workgroup barrier and bumps the counter with a
// relaxed agent-scope atomic; readers use agent-scope loads. A build with -DTR_FORMAL_FENCES adds
// the memory model's agent-scope release fence before the counter atomic and acquire fence after
// it in the last arriver (buffer_wbl2 / buffer_inv on gfx950), for measuring what they cost.
__device__ __forceinline__ void handoff_release() {
#ifdef TR_FORMAL_FENCES
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
#endif
}
__device__ __forceinline__ void handoff_acquire() {
#ifdef TR_FORMAL_FENCES
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
#endif
}

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16, round to nearest even, NaN kept a quiet NaN (what torch's .to(bfloat16) does):
// gfx950's v_cvt_pk_bf16_f32, one instruction for two values. Its result equals the bit-level
// rounding (u + 0x7fff + bit 16 of u, then the high half; a NaN's high half with bit 6 set) on
// every one of the 2^32 fp32 inputs, checked on the device.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// fp16 bits -> fp32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)b);
}

// silu(g) * u in fp32, the MLP activation (tokenrush/fused.py:76). One definition for the fused
// GEMM epilogue and the stand-alone kernel, so the two paths agree bit for bit.
__device__ __forceinline__ float silu_mul_f32(float g, float u) { return g / (1.0f + __expf(-g)) * u; }

// 8 bf16 (one 16-byte load) <-> fp32.
__device__ __forceinline__ void unpack8(const uint4& u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_bits_to_f32(w[i] & 0xFFFFu);
    f[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
  }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = f32x2_to_bf16x2_bits(f[2 * i], f[2 * i + 1]);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Pieces of the residual RMSNorm (tokenrush/fused.py:23-60) shared by add_rmsnorm_kernel and the
// GEMM's norm epilogue, so that the two paths give the same bits whatever each file's
// contraction flags: the residual bf16(x + bf16(h)), the inverse RMS from a row's sum of
// squares, and the gain ((1 + w), or the plain w * bf16(x * r)).
__device__ __forceinline__ float resid_add(float x, float h) {
#pragma clang fp contract(off)
  return bf16_bits_to_f32(f32_to_bf16_bits(x + bf16_bits_to_f32(f32_to_bf16_bits(h))));
}
__device__ __forceinline__ float rms_inv(float ss, int N, float eps) {
#pragma clang fp contract(off)
  return 1.0f / sqrtf(ss / (float)N + eps);
}
__device__ __forceinline__ float rms_apply(float v, float r, float w, int plain) {
#pragma clang fp contract(off)
  return plain ? w * bf16_bits_to_f32(f32_to_bf16_bits(v * r)) : v * r * (1.0f + w);
}
// Sum of squares of 8 consecutive elements, in element order.
__device__ __forceinline__ float ssq8(const float (&v)[8]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = fmaf(v[e], v[e], ss);
  return ss;
}

// A value the compiler must keep in a VGPR: lets v_and_or_b32 take (VGPR, SGPR, VGPR)
// operands, since a gfx9 VOP3 instruction reads at most one scalar/literal.
__device__ __forceinline__ uint32_t vgpr_const(uint32_t c) {
  uint32_t r;
  asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(c));
  return r;
}

// A workgroup barrier that orders LDS accesses only. __syncthreads' workgroup fence also makes
// the wave wait for its global memory operations still in flight (loads issued ahead, stores
// not yet acknowledged), which a barrier guarding LDS alone does not need.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Cross-lane sums on the VALU (DPP and the gfx950 permlane swaps) instead of LDS-routed
// ds_bpermute shuffles. Each returns, in every lane, the sum over the lanes of its group; the
// two lanes of a pair add the same two values (a + b == b + a), so every lane of a group ends
// with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// lanes l and l ^ 8 (row_ror:8 inside each 16-lane row)
__device__ __forceinline__ float sum_x8(float v) { return v + dpp_mov<0x128>(v); }
// lanes l and l ^ 16: v_permlane16_swap leaves (row 2i, row 2i) in one result and
// (row 2i + 1, row 2i + 1) in the other
__device__ __forceinline__ float sum_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// lanes l and l ^ 32
__device__ __forceinline__ float sum_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Four sums over the lanes l, l ^ 8, l ^ 16, l ^ 32 at once. A permlane swap exchanges the odd
// rows (halves) of one register with the even rows (halves) of another, so one swap and one add
// reduce two values at a time: a's pair sums land in the even rows and b's in the odd ones, then
// the two results' halves are combined the same way. Each lane returns one total: a in row 0
// (lanes 0-15), b in row 1, c in row 2, d in row 3. Every total is added in the same order as
// sum_x32(sum_x16(sum_x8(v))) adds it, so it has the same bits.
__device__ __forceinline__ float sum_x8_16_32_4(float a, float b, float c, float d) {
  a = sum_x8(a);
  b = sum_x8(b);
  c = sum_x8(c);
  d = sum_x8(d);
  const auto r1 = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const auto r2 = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(d), false, false);
  const float ab = __uint_as_float(r1[0]) + __uint_as_float(r1[1]);
  const float cd = __uint_as_float(r2[0]) + __uint_as_float(r2[1]);
  const auto r3 = __builtin_amdgcn_permlane32_swap(__float_as_uint(ab), __float_as_uint(cd), false, false);
  return __uint_as_float(r3[0]) + __uint_as_float(r3[1]);
}
// the 32 lanes of the same parity (l % 2): quad xor 2, row_ror 4, row_ror 8, row pairs, halves
__device__ __forceinline__ float sum_parity(float v) {
  v = v + dpp_mov<0x4E>(v);
  v = v + dpp_mov<0x124>(v);
  v = sum_x8(v);
  return sum_x32(sum_x16(v));
}
// all 64 lanes: quad xor 1, quad xor 2, row_ror 4, row_ror 8, then the row pairs and halves
__device__ __forceinline__ float sum_wave(float v) {
  v = v + dpp_mov<0xB1>(v);
  v = v + dpp_mov<0x4E>(v);
  v = v + dpp_mov<0x124>(v);
  v = sum_x8(v);
  return sum_x32(sum_x16(v));
}

}  // namespace tr
