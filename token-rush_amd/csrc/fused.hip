// Row kernels around the verify GEMMs: the split-K partial consumer (residual add + RMSNorm)
// and the MLP activation. Restated from the reference's Triton kernels (tokenrush/fused.py).
//
// add_rmsnorm (tokenrush/fused.py:23-60): for each row t,
//   h   = sum over slots s of partials[s, t, :] in slot order (fp32), rounded to bf16
//         (or h given as bf16, or no h)
//   x'  = bf16(x + h)            the residual stream, written to xo
//   y   = x' * rsqrt(mean(x'^2) + eps) * (1 + w)      (plain: bf16(w * bf16(x' * rsqrt(...))))
// One workgroup per row; the row stays in registers between the two passes.
//
// silu_mul (tokenrush/fused.py:67-87): y[t, i] = silu(gate[t, i]) * up[t, i] with gate_up[t] =
// [gate (F) | up (F)] (rows ld elements apart), fp32 arithmetic, bf16 out.
#include "tr_common.h"

namespace tr {

constexpr int kNormThreads = 1024;
constexpr int kNormPerThread = 8;  // N <= 8192

enum { H_NONE = 0, H_BF16 = 1, H_PARTIALS = 2 };

__device__ __forceinline__ float block_sum(float v, float* sh) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  float t = 0.f;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) t += sh[w];  // same order in every thread
  return t;
}

__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(const uint16_t* __restrict__ x, const void* h,
                                                                   int h_mode, int S, const uint16_t* __restrict__ w,
                                                                   uint16_t* xo, uint16_t* __restrict__ y, int T, int N,
                                                                   float eps, int plain) {
  __shared__ float sh[kNormThreads / 64];
  const int t = blockIdx.x;
  float v[kNormPerThread];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kNormPerThread; ++j) {
    const int i = threadIdx.x + j * blockDim.x;
    float xv = 0.f;
    if (i < N) {
      xv = bf16_bits_to_f32(x[(size_t)t * N + i]);
      if (h_mode != H_NONE) {
        float hv;
        if (h_mode == H_BF16) {
          hv = bf16_bits_to_f32(((const uint16_t*)h)[(size_t)t * N + i]);
        } else {
          const float* p = (const float*)h;
          hv = p[(size_t)t * N + i];
          for (int s = 1; s < S; ++s) hv += p[((size_t)s * T + t) * N + i];
          hv = bf16_bits_to_f32(f32_to_bf16_bits(hv));
        }
        xv = bf16_bits_to_f32(f32_to_bf16_bits(xv + hv));  // the residual stream is bf16
        xo[(size_t)t * N + i] = f32_to_bf16_bits(xv);
      }
    }
    v[j] = xv;
    ss = fmaf(xv, xv, ss);
  }
  const float var = block_sum(ss, sh) / (float)N;
  const float r = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < kNormPerThread; ++j) {
    const int i = threadIdx.x + j * blockDim.x;
    if (i >= N) continue;
    const float wv = bf16_bits_to_f32(w[i]);
    float out;
    if (plain)
      out = wv * bf16_bits_to_f32(f32_to_bf16_bits(v[j] * r));  // Qwen3: cast, then weight * x
    else
      out = v[j] * r * (1.0f + wv);                             // Qwen3.5: gain is 1 + weight
    y[(size_t)t * N + i] = f32_to_bf16_bits(out);
  }
}

__global__ void silu_mul_kernel(const uint16_t* __restrict__ gu, long ld, uint16_t* __restrict__ y, int T, int F) {
  const size_t total = (size_t)T * F;
  for (size_t e = blockIdx.x * (size_t)blockDim.x + threadIdx.x; e < total; e += (size_t)gridDim.x * blockDim.x) {
    const size_t t = e / F, i = e % F;
    const float g = bf16_bits_to_f32(gu[t * ld + i]);
    const float u = bf16_bits_to_f32(gu[t * ld + F + i]);
    y[e] = f32_to_bf16_bits(g / (1.0f + expf(-g)) * u);
  }
}

}  // namespace tr

using namespace tr;

extern "C" {

int tr_add_rmsnorm(const void* x, const void* h, int h_mode, int n_slots, const void* weight, void* xo, void* y,
                   int T, int N, float eps, int plain, void* stream) {
  if (!x || !weight || !y) return TR_ERR_ARG;
  if (h_mode < H_NONE || h_mode > H_PARTIALS || (h_mode != H_NONE && (!h || !xo))) return TR_ERR_ARG;
  if (h_mode == H_PARTIALS && n_slots < 1) return TR_ERR_ARG;
  if (T < 0 || N <= 0 || N > kNormThreads * kNormPerThread) return TR_ERR_SHAPE;
  if (T == 0) return TR_OK;
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(T), dim3(kNormThreads), 0, (hipStream_t)stream, (const uint16_t*)x, h,
                     h_mode, n_slots, (const uint16_t*)weight, (uint16_t*)xo, (uint16_t*)y, T, N, eps, plain);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_silu_mul(const void* gate_up, long ld, void* y, int T, int F, void* stream) {
  if (!gate_up || !y) return TR_ERR_ARG;
  if (T < 0 || F <= 0) return TR_ERR_SHAPE;
  if (ld == 0) ld = 2L * F;
  if (ld < 2L * F) return TR_ERR_ARG;
  if (T == 0) return TR_OK;
  size_t blocks = ((size_t)T * F + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((int)blocks), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)gate_up,
                     ld, (uint16_t*)y, T, F);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"
