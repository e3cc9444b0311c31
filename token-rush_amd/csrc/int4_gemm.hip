// int4 group-128 (scale + min) verify GEMM for gfx950.
//
// y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k/128] + mn[n, k/128]),  m < M <= 32.
//
// The reference computes this with a Marlin port (tokenrush/csrc/marlin_bf16.cu:145-581) or,
// for M = 1, with the fold  s * sum(q x) + m * sum(x)  per (row, group)
// (tokenrush/quant.py:113-119). This kernel uses the fold on the matrix cores:
//
//   * Codes stay integers. A nibble q becomes the bf16 value 128 + q with one v_and_or_b32
//     (exponent of 128, q in the low mantissa bits), so no multiply touches a weight.
//   * v_mfma_f32_16x16x32_bf16 contracts 16 activation rows (A) against 16 weight rows (B)
//     over 32 k: E = sum x (128 + q) per group, fp32.
//   * One more MFMA chain against a ones operand gives sum(x) per row and group, and the
//     group result is  s * E + (mn - 128 s) * sum(x)  in fp32, applied once per group.
//
// Rows of x beyond M are zero lanes, so every output row is computed by the same
// instructions whatever M is: row i of an M = 1 call is bit-identical to row i of an
// M = 8 call (the property tests/test_marlin.py:42-52 of the reference checks).
//
// Weight layout ("strip layout", made once at load time by tr_pack_int4):
//   codes[N/16][G][64 lanes][16 B]: one 1 KiB tile per (16-row strip, group). Lane l holds
//   row l%16, k in [32*(l/16), 32*(l/16)+32) of the group, as four 32-bit words; word j
//   covers k0 = 32*(l/16) + 8j .. k0+7 with code k0+2p in nibble p and k0+2p+1 in nibble
//   p+4 (p = 0..3), so (w >> 4p) & 0x000F000F is the bf16 pair (k0+2p, k0+2p+1).
//   A wave's 16-byte load of a tile is one contiguous, fully coalesced 1 KiB read, and
//   a strip's tiles are contiguous along K.
//   scale, mn: the engine's own [N, K/128] arrays (bf16, or fp16 for the benchmark
//   format), read in place.
//
// Work split: a workgroup owns T strips (16T rows) and one K slice (slot); its W waves
// split the slot's groups evenly and reduce through LDS in fixed wave order, so results
// are deterministic. With S > 1 slots each slot writes its own fp32 partial [S, M, N]
// (no locks, no atomics), the contract of the reference's partials()
// (tokenrush/quant.py:381-391, tokenrush/marlin.py:158-168).
#include "tr_common.h"

namespace tr {

constexpr int kGroup = 128;

template <int T, int MT>
struct Stage {
  uint4 w[T];        // code tile words, one 16-B chunk per strip
  uint32_t s[T];     // raw 16-bit scale of (row, group)
  uint32_t m[T];     // raw 16-bit min of (row, group)
  uint4 x[MT][4];    // activation chunks: row 16*mt + lane%16, 32 k of this lane's quad
};

template <int T, int MT>
__device__ __forceinline__ void load_stage(Stage<T, MT>& st, const uint4* __restrict__ codes,
                                           const uint16_t* __restrict__ scale,
                                           const uint16_t* __restrict__ mn,
                                           const uint16_t* __restrict__ x, int strip0, int G, int g,
                                           int lane, int M, int K) {
#pragma unroll
  for (int t = 0; t < T; ++t) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4* p = (const u32x4*)(codes + ((size_t)(strip0 + t) * G + g) * 64 + lane);
    const u32x4 v = __builtin_nontemporal_load(p);
    st.w[t] = make_uint4(v.x, v.y, v.z, v.w);
    size_t row = (size_t)(strip0 + t) * 16 + (lane & 15);
    st.s[t] = scale[row * G + g];
    st.m[t] = mn[row * G + g];
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    int xr = 16 * mt + (lane & 15);
    if (xr < M) {
      const uint4* p = (const uint4*)(x + (size_t)xr * K + g * kGroup + 32 * (lane >> 4));
#pragma unroll
      for (int j = 0; j < 4; ++j) st.x[mt][j] = p[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) st.x[mt][j] = make_uint4(0, 0, 0, 0);
    }
  }
}

template <int T, int MT, bool F16S>
__device__ __forceinline__ void compute_stage(const Stage<T, MT>& st, f32x4 (&acc)[T][MT],
                                              uint32_t kExp128, uint32_t kOnes) {
  const uint32_t kMask = 0x000F000Fu;
  const uint4 ones4 = make_uint4(kOnes, kOnes, kOnes, kOnes);
  const bf16x8 ones = __builtin_bit_cast(bf16x8, ones4);
  f32x4 X[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    X[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      X[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[mt][j]), ones,
                                                      X[mt], 0, 0, 0);
  }
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t wd[4] = {st.w[t].x, st.w[t].y, st.w[t].z, st.w[t].w};
    bf16x8 b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint4 d;
      d.x = (wd[j] & kMask) | kExp128;
      d.y = ((wd[j] >> 4) & kMask) | kExp128;
      d.z = ((wd[j] >> 8) & kMask) | kExp128;
      d.w = ((wd[j] >> 12) & kMask) | kExp128;
      b[j] = __builtin_bit_cast(bf16x8, d);
    }
    float sf, mf;
    if (F16S) {
      sf = f16_bits_to_f32(st.s[t]);
      mf = f16_bits_to_f32(st.m[t]);
    } else {
      sf = bf16_bits_to_f32(st.s[t]);
      mf = bf16_bits_to_f32(st.m[t]);
    }
    const float c1 = fmaf(-128.f, sf, mf);  // mn - 128 s: removes the +128 code offset
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      f32x4 E = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        E = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.x[mt][j]), b[j], E,
                                                    0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[t][mt][r] = fmaf(sf, E[r], acc[t][mt][r]);
        acc[t][mt][r] = fmaf(c1, X[mt][r], acc[t][mt][r]);
      }
    }
  }
}

// One output element of the wave tile: accumulator (t, mt, r) of lane l is
// y[m = 16 mt + 4 (l/16) + r, n = 16 (strip0 + t) + l%16].
__device__ __forceinline__ void store_out(void* out, bool partial, int slot, int M, int N, int m, int n,
                                          float v) {
  if (m >= M) return;
  if (partial)
    ((float*)out)[((size_t)slot * M + m) * N + n] = v;
  else
    ((uint16_t*)out)[(size_t)m * N + n] = f32_to_bf16_bits(v);
}

template <int T, int MT, bool F16S, int P>
__global__ __launch_bounds__(512) void int4_gemm_kernel(const uint16_t* __restrict__ x,
                                                         const uint4* __restrict__ codes,
                                                         const uint16_t* __restrict__ scale,
                                                         const uint16_t* __restrict__ mn,
                                                         void* __restrict__ out, int M, int N, int K,
                                                         int S, int partial) {
  extern __shared__ float red[];
  const int G = K / kGroup;
  const int W = blockDim.x >> 6;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nrb = N / (16 * T);
  const int rb = blockIdx.x % nrb;
  const int slot = blockIdx.x / nrb;
  const int strip0 = rb * T;

  const int gs0 = (int)(((long)slot * G) / S), gs1 = (int)(((long)(slot + 1) * G) / S);
  const int len = gs1 - gs0;
  const int g0 = gs0 + (wave * len) / W, g1 = gs0 + ((wave + 1) * len) / W;

  const uint32_t kExp128 = vgpr_const(0x43004300u);
  const uint32_t kOnes = 0x3F803F80u;

  f32x4 acc[T][MT];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  Stage<T, MT> st[P];
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (g0 + p < g1) load_stage<T, MT>(st[p], codes, scale, mn, x, strip0, G, g0 + p, lane, M, K);

  for (int gb = g0; gb < g1; gb += P) {
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int g = gb + p;
      if (g < g1) {
        compute_stage<T, MT, F16S>(st[p], acc, kExp128, kOnes);
        if (g + P < g1) load_stage<T, MT>(st[p], codes, scale, mn, x, strip0, G, g + P, lane, M, K);
      }
    }
  }

  constexpr int Q = T * MT * 4;  // accumulators per lane
  if (W == 1) {
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          store_out(out, partial, slot, M, N, 16 * mt + 4 * (lane >> 4) + r, 16 * (strip0 + t) + (lane & 15),
                    acc[t][mt][r]);
    return;
  }
  // Cross-wave reduction in fixed wave order: red[w][q][lane].
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wave * Q + (t * MT + mt) * 4 + r) * 64 + lane] = acc[t][mt][r];
  __syncthreads();
  for (int e = threadIdx.x; e < Q * 64; e += blockDim.x) {
    const int q = e >> 6, l = e & 63;
    float v = red[e];
    for (int w = 1; w < W; ++w) v += red[w * Q * 64 + e];
    const int r = q & 3, mt = (q >> 2) % MT, t = (q >> 2) / MT;
    store_out(out, partial, slot, M, N, 16 * mt + 4 * (l >> 4) + r, 16 * (strip0 + t) + (l & 15), v);
  }
}

// ----------------------------------------------------------------------------- layout kernels

// Engine packing (uint8 [N, K/2], element 2j in the low nibble of byte j; tokenrush/quant.py:9-10)
// -> strip layout. One thread per output 32-bit word.
__global__ void pack_kernel(const uint32_t* __restrict__ q, uint32_t* __restrict__ codes, int N, int K) {
  const int G = K / kGroup;
  const size_t total = (size_t)N / 16 * G * 256;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int j = i & 3, lane = (i >> 2) & 63;
    const size_t tile = i >> 8;
    const int g = tile % G;
    const size_t strip = tile / G;
    const size_t n = strip * 16 + (lane & 15);
    const int k0 = g * kGroup + 32 * (lane >> 4) + 8 * j;
    const uint32_t u = q[(n * K + k0) / 8];  // bytes b0..b3 = codes k0..k0+7
    uint32_t w = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t b = (u >> (8 * p)) & 0xFF;
      w |= (b & 0xF) << (4 * p);
      w |= (b >> 4) << (16 + 4 * p);
    }
    codes[i] = w;
  }
}

// Strip layout -> engine packing (the inverse of pack_kernel).
__global__ void unpack_kernel(const uint32_t* __restrict__ codes, uint32_t* __restrict__ q, int N, int K) {
  const int G = K / kGroup;
  const size_t total = (size_t)N / 16 * G * 256;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int j = i & 3, lane = (i >> 2) & 63;
    const size_t tile = i >> 8;
    const int g = tile % G;
    const size_t strip = tile / G;
    const size_t n = strip * 16 + (lane & 15);
    const int k0 = g * kGroup + 32 * (lane >> 4) + 8 * j;
    const uint32_t w = codes[i];
    uint32_t u = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t lo = (w >> (4 * p)) & 0xF, hi = (w >> (16 + 4 * p)) & 0xF;
      u |= (lo | (hi << 4)) << (8 * p);
    }
    q[(n * K + k0) / 8] = u;
  }
}

// dequantize_int4 (tokenrush/quant.py:47-53): w = bf16(bf16(q * s) + m), two roundings, from the
// engine packing. One thread per pair of elements (one byte).
template <bool F16S>
__global__ void dequant_kernel(const uint8_t* __restrict__ q, const uint16_t* __restrict__ scale,
                               const uint16_t* __restrict__ mn, uint32_t* __restrict__ out, int N, int K) {
  const int G = K / kGroup;
  const size_t total = (size_t)N * K / 2;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const size_t n = i / (K / 2);
    const int k = (int)(i % (K / 2)) * 2;
    const size_t gi = n * G + k / kGroup;
    // bf16 parameters: torch's in-place bf16 mul then add. fp16 parameters (the benchmark
    // format): the same two roundings in fp16, output fp16.
    const float s = F16S ? f16_bits_to_f32(scale[gi]) : bf16_bits_to_f32(scale[gi]);
    const float m = F16S ? f16_bits_to_f32(mn[gi]) : bf16_bits_to_f32(mn[gi]);
    const uint32_t b = q[i];
    uint32_t r = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float code = (float)((b >> (4 * h)) & 0xF);
      uint32_t bits;
      if (F16S) {
        const float t = (float)(_Float16)(code * s);
        bits = __builtin_bit_cast(uint16_t, (_Float16)(t + m));
      } else {
        const float t = bf16_bits_to_f32(f32_to_bf16_bits(code * s));
        bits = f32_to_bf16_bits(t + m);
      }
      r |= bits << (16 * h);
    }
    out[i] = r;
  }
}

}  // namespace tr

// ----------------------------------------------------------------------------- C ABI
using namespace tr;

namespace {

template <int T, int MT, bool F16S>
hipError_t launch_t(const void* x, const void* codes, const void* scale, const void* mn, void* out, int M,
                    int N, int K, int S, int W, int partial, hipStream_t stream) {
  const int nrb = N / (16 * T);
  const dim3 grid(nrb * S), block(64 * W);
  const size_t lds = W > 1 ? (size_t)W * T * MT * 4 * 64 * sizeof(float) : 0;
  hipLaunchKernelGGL((int4_gemm_kernel<T, MT, F16S, 3>), grid, block, lds, stream, (const uint16_t*)x,
                     (const uint4*)codes, (const uint16_t*)scale, (const uint16_t*)mn, out, M, N, K, S, partial);
  return hipGetLastError();
}

template <bool F16S>
hipError_t launch_s(int T, int MT, const void* x, const void* codes, const void* scale, const void* mn, void* out,
                    int M, int N, int K, int S, int W, int partial, hipStream_t stream) {
#define TR_CASE(TT, MM) \
  if (T == TT && MT == MM) return launch_t<TT, MM, F16S>(x, codes, scale, mn, out, M, N, K, S, W, partial, stream);
  TR_CASE(1, 1) TR_CASE(2, 1) TR_CASE(4, 1) TR_CASE(1, 2) TR_CASE(2, 2)
#undef TR_CASE
  return hipErrorInvalidValue;
}

}  // namespace

extern "C" {

// Default tiling for an N x K weight. Independent of M, so every row of the output is
// computed identically for every M (see the file comment).
int tr_gemm_plan(int N, int K, int* T, int* W, int* S) {
  if (N <= 0 || K <= 0 || N % 16 || K % kGroup || !T || !W || !S) return TR_ERR_SHAPE;
  const int strips = N / 16, G = K / kGroup;
  int t = 1;
  if (strips % 2 == 0 && strips / 2 >= 512) t = 2;
  const int nrb = strips / t;
  int w = (6144 + nrb - 1) / nrb;     // aim at ~6k waves over the 256 CUs
  int wmax = G / 3 > 0 ? G / 3 : 1;   // keep >= 3 groups per wave
  if (w > wmax) w = wmax;
  if (w > 8) w = 8;
  if (w < 1) w = 1;
  *T = t;
  *W = w;
  *S = 1;
  return TR_OK;
}

int tr_partial_slots(int N, int K, int M) {
  (void)M;
  int T, W, S;
  if (tr_gemm_plan(N, K, &T, &W, &S)) return -1;
  return S;
}

int tr_int4_gemm_ex(const void* x, const void* packed, const void* scale, const void* mn, void* out,
                    void* partials, int M, int N, int K, int group, int scale_dtype, int n_slots, int T, int W,
                    void* stream) {
  if (group != kGroup) return TR_ERR_CONFIG;
  if (M < 0 || M > 32 || N <= 0 || K <= 0 || N % 16 || K % kGroup) return TR_ERR_SHAPE;
  if (M == 0) return TR_OK;
  if (!x || !packed || !scale || !mn || (!out == !partials)) return TR_ERR_ARG;
  if (scale_dtype != 0 && scale_dtype != 1) return TR_ERR_ARG;
  if (T != 1 && T != 2 && T != 4) return TR_ERR_CONFIG;
  if ((N / 16) % T) return TR_ERR_CONFIG;
  if (T == 4 && M > 16) return TR_ERR_CONFIG;
  if (W < 1 || W > 8) return TR_ERR_CONFIG;
  const int partial = partials != nullptr;
  int S = 1;
  if (partial) {
    if (n_slots < 1 || n_slots > K / kGroup) return TR_ERR_CONFIG;
    S = n_slots;
  }
  const int MT = M > 16 ? 2 : 1;
  hipError_t e = scale_dtype == 1
                     ? launch_s<true>(T, MT, x, packed, scale, mn, partial ? partials : out, M, N, K, S, W, partial,
                                      (hipStream_t)stream)
                     : launch_s<false>(T, MT, x, packed, scale, mn, partial ? partials : out, M, N, K, S, W,
                                       partial, (hipStream_t)stream);
  return e == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_int4_gemm(const void* x, const void* packed, const void* scale, const void* mn, void* out, void* partials,
                 int M, int N, int K, int group, int scale_dtype, int n_slots, void* stream) {
  int T, W, S;
  int rc = tr_gemm_plan(N, K, &T, &W, &S);
  if (rc) return rc;
  return tr_int4_gemm_ex(x, packed, scale, mn, out, partials, M, N, K, group, scale_dtype, n_slots, T, W, stream);
}

static int grid_for(size_t work) {
  size_t b = (work + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return (int)b;
}

int tr_pack_int4(const void* qweight, void* packed, int N, int K, void* stream) {
  if (!qweight || !packed) return TR_ERR_ARG;
  if (N <= 0 || K <= 0 || N % 16 || K % kGroup) return TR_ERR_SHAPE;
  const size_t total = (size_t)N / 16 * (K / kGroup) * 256;
  hipLaunchKernelGGL(pack_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, (const uint32_t*)qweight,
                     (uint32_t*)packed, N, K);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_unpack_int4(const void* packed, void* qweight, int N, int K, void* stream) {
  if (!qweight || !packed) return TR_ERR_ARG;
  if (N <= 0 || K <= 0 || N % 16 || K % kGroup) return TR_ERR_SHAPE;
  const size_t total = (size_t)N / 16 * (K / kGroup) * 256;
  hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)packed, (uint32_t*)qweight, N, K);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_dequant_int4(const void* qweight, const void* scale, const void* mn, void* out, int N, int K, int group,
                    int scale_dtype, void* stream) {
  if (!qweight || !scale || !mn || !out) return TR_ERR_ARG;
  if (group != kGroup) return TR_ERR_CONFIG;
  if (N <= 0 || K <= 0 || K % kGroup) return TR_ERR_SHAPE;
  const size_t total = (size_t)N * K / 2;
  if (scale_dtype == 1)
    hipLaunchKernelGGL(dequant_kernel<true>, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)qweight, (const uint16_t*)scale, (const uint16_t*)mn, (uint32_t*)out, N, K);
  else if (scale_dtype == 0)
    hipLaunchKernelGGL(dequant_kernel<false>, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                       (const uint8_t*)qweight, (const uint16_t*)scale, (const uint16_t*)mn, (uint32_t*)out, N, K);
  else
    return TR_ERR_ARG;
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"
