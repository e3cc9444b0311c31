// Row kernels around the verify GEMMs: the split-K partial consumer (residual add + RMSNorm)
// and the MLP activation. Restated from the reference's Triton kernels (tokenrush/fused.py).
//
// add_rmsnorm (tokenrush/fused.py:23-60): for each row t,
//   h   = sum over slots s of partials[s, t, :] in slot order (fp32), rounded to bf16
//         (or h given as bf16, or no h)
//   x'  = bf16(x + h)            the residual stream, written to xo
//   y   = x' * rsqrt(mean(x'^2) + eps) * (1 + w)      (plain: bf16(w * bf16(x' * rsqrt(...))))
// One workgroup per row, 8 elements per thread in registers between the two passes; N % 8 == 0,
// N <= 8192, at most 8 partial slots.
//
// embed_rows (tokenrush/model.py:215, x = embed[tokens]): out[t] = table[ids[t]], bf16 rows.
//
// silu_mul (tokenrush/fused.py:67-87): y[t, i] = silu(gate[t, i]) * up[t, i] with gate_up[t] =
// [gate (F) | up (F)] (rows ld elements apart), fp32 arithmetic, bf16 out.
#include "tr_common.h"

namespace tr {

constexpr int kRowVec = 8;          // elements per thread: one 16-byte bf16 load
constexpr int kMaxRowThreads = 1024;
constexpr int kMaxSlots = 8;        // split-K slots the consumer sums (the GEMM makes <= 4 here)

enum { H_NONE = 0, H_BF16 = 1, H_PARTIALS = 2 };

typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Sum over the workgroup: each wave's lanes by sum_wave, then the waves in index order (the same
// order in every thread, and the order of the GEMM's norm epilogue).
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = sum_wave(v);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) sh[wave] = v;
  __syncthreads();
  float t = 0.f;
  const int nw = blockDim.x >> 6;
  for (int w = 0; w < nw; ++w) t += sh[w];
  return t;
}

// One workgroup per row, 8 consecutive elements per thread, every load of the row (x, all S
// partial slots and the gain) issued before any arithmetic.
template <int HM, int S>
__global__ __launch_bounds__(kMaxRowThreads) void add_rmsnorm_kernel(const uint16_t* __restrict__ x, const void* h,
                                                                     const uint16_t* __restrict__ w, uint16_t* xo,
                                                                     uint16_t* __restrict__ y, int T, int N, float eps,
                                                                     int plain) {
  __shared__ float sh[kMaxRowThreads / 64];
  const int t = blockIdx.x;
  const int i0 = threadIdx.x * kRowVec;
  const bool on = i0 < N;
  const size_t row = (size_t)t * N + i0;
  float v[kRowVec];
  uint4 xv = make_uint4(0, 0, 0, 0), hv = xv, wv = xv;
  float4 part[S > 0 ? S : 1][2];
#pragma unroll
  for (int s = 0; s < (S > 0 ? S : 1); ++s) part[s][0] = part[s][1] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (on) {
    xv = *(const uint4*)(x + row);
    wv = *(const uint4*)(w + i0);
    if (HM == H_BF16) hv = *(const uint4*)((const uint16_t*)h + row);
    if (HM == H_PARTIALS) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const float4* p = (const float4*)((const float*)h + ((size_t)s * T + t) * N + i0);
        part[s][0] = p[0];
        part[s][1] = p[1];
      }
    }
  }
  unpack8(xv, v);
  if (HM != H_NONE) {
    float hf[kRowVec];
    if (HM == H_BF16) {
      unpack8(hv, hf);
    } else {
#pragma unroll
      for (int e = 0; e < kRowVec; ++e) {
        float acc = e < 4 ? part[0][0][e] : part[0][1][e - 4];
#pragma unroll
        for (int s = 1; s < S; ++s) acc += e < 4 ? part[s][0][e] : part[s][1][e - 4];  // slot order
        hf[e] = acc;
      }
    }
#pragma unroll
    for (int e = 0; e < kRowVec; ++e) v[e] = resid_add(v[e], hf[e]);  // bf16(x + bf16(h))
    if (on) *(uint4*)(xo + row) = pack8(v);
  }
  const float r = rms_inv(block_sum(ssq8(v), sh), N, eps);
  if (!on) return;
  float wf[kRowVec], out[kRowVec];
  unpack8(wv, wf);
#pragma unroll
  for (int e = 0; e < kRowVec; ++e) out[e] = rms_apply(v[e], r, wf[e], plain);  // Qwen3.5 (1 + w) or Qwen3 plain
  *(uint4*)(y + row) = pack8(out);
}

// Grid (F / (8 * blockDim), T): 8 consecutive elements per thread.
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, long ld, uint16_t* __restrict__ y,
                                                       int F) {
  const int t = blockIdx.y;
  const int i0 = (blockIdx.x * blockDim.x + threadIdx.x) * kRowVec;
  if (i0 >= F) return;
  float g[kRowVec], u[kRowVec], out[kRowVec];
  unpack8(*(const uint4*)(gu + (size_t)t * ld + i0), g);
  unpack8(*(const uint4*)(gu + (size_t)t * ld + F + i0), u);
#pragma unroll
  for (int e = 0; e < kRowVec; ++e) out[e] = silu_mul_f32(g[e], u[e]);
  *(uint4*)(y + (size_t)t * F + i0) = pack8(out);
}

// One 16-byte vector per thread; grid (row chunks, T). An id outside [0, V) writes a zero row and
// sets *status to 1 (the reference's indexing would raise; a device kernel can only report).
__global__ void embed_rows_kernel(const uint16_t* __restrict__ table, const int64_t* __restrict__ ids,
                                  uint16_t* __restrict__ out, int H, long V, int* status) {
  const int t = blockIdx.y;
  const int i = (blockIdx.x * blockDim.x + threadIdx.x) * kRowVec;
  if (i >= H) return;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < V;
  const uint4 v = ok ? *(const uint4*)(table + (size_t)id * H + i) : make_uint4(0u, 0u, 0u, 0u);
  *(uint4*)(out + (size_t)t * H + i) = v;
  if (!ok && i == 0 && status) *status = 1;
}

}  // namespace tr

using namespace tr;

template <int HM, int S>
static hipError_t launch_norm(dim3 grid, dim3 block, hipStream_t st, const void* x, const void* h, const void* w,
                              void* xo, void* y, int T, int N, float eps, int plain) {
  hipLaunchKernelGGL((add_rmsnorm_kernel<HM, S>), grid, block, 0, st, (const uint16_t*)x, h, (const uint16_t*)w,
                     (uint16_t*)xo, (uint16_t*)y, T, N, eps, plain);
  return hipGetLastError();
}

extern "C" {

int tr_add_rmsnorm(const void* x, const void* h, int h_mode, int n_slots, const void* weight, void* xo, void* y,
                   int T, int N, float eps, int plain, void* stream) {
  if (!x || !weight || !y) return TR_ERR_ARG;
  if (h_mode < H_NONE || h_mode > H_PARTIALS || (h_mode != H_NONE && (!h || !xo))) return TR_ERR_ARG;
  if (h_mode == H_PARTIALS && (n_slots < 1 || n_slots > kMaxSlots)) return TR_ERR_ARG;
  if (T < 0 || N <= 0 || N % kRowVec || N > kMaxRowThreads * kRowVec) return TR_ERR_SHAPE;
  if (T == 0) return TR_OK;
  const int threads = ((N / kRowVec + 63) / 64) * 64;
  const dim3 grid(T), block(threads);
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (h_mode == H_NONE) e = launch_norm<H_NONE, 0>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain);
  else if (h_mode == H_BF16) e = launch_norm<H_BF16, 0>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain);
  else {
    switch (n_slots) {
      case 1: e = launch_norm<H_PARTIALS, 1>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      case 2: e = launch_norm<H_PARTIALS, 2>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      case 3: e = launch_norm<H_PARTIALS, 3>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      case 4: e = launch_norm<H_PARTIALS, 4>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      case 5: e = launch_norm<H_PARTIALS, 5>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      case 6: e = launch_norm<H_PARTIALS, 6>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      case 7: e = launch_norm<H_PARTIALS, 7>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
      default: e = launch_norm<H_PARTIALS, 8>(grid, block, st, x, h, weight, xo, y, T, N, eps, plain); break;
    }
  }
  return e == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_embed_rows(const void* table, const int64_t* ids, void* out, int T, int H, long V, int* status,
                  void* stream) {
  if (!table || !ids || !out) return TR_ERR_ARG;
  if (T < 0 || H <= 0 || H % kRowVec || V <= 0) return TR_ERR_SHAPE;
  if (T == 0) return TR_OK;
  const int per_block = 256 * kRowVec;
  hipLaunchKernelGGL(embed_rows_kernel, dim3((H + per_block - 1) / per_block, T), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)table, ids, (uint16_t*)out, H, V, status);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_silu_mul(const void* gate_up, long ld, void* y, int T, int F, void* stream) {
  if (!gate_up || !y) return TR_ERR_ARG;
  if (T < 0 || F <= 0 || F % kRowVec) return TR_ERR_SHAPE;
  if (ld == 0) ld = 2L * F;
  if (ld < 2L * F || ld % kRowVec) return TR_ERR_ARG;
  if (T == 0) return TR_OK;
  const int per_block = 256 * kRowVec;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((F + per_block - 1) / per_block, T), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)gate_up, ld, (uint16_t*)y, F);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"
