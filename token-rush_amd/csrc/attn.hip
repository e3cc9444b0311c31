// Full-attention verify step for gfx950 over an FP8 (e4m3fn) KV cache with per-(head, position)
// fp32 scales: the prep of the M new tokens (q/k RMSNorm, partial rope, cache write) and
// flash-decoding (split over the live keys, then a reduce with the sigmoid output gate).
//
// Follows the reference's Triton kernels (tokenrush/fused.py:247-325 _attn_prep_kernel and
// attn_prep, :355-470 _attn_split_kernel, _attn_reduce_kernel and attn_decode_fused):
//   prep (heads 0..HQ-1 from the q part of qkv [HQ (q | gate) 2D | HKV D | HKV D], heads HQ..
//   for k): xn = bf16(x * rsqrt(mean(x^2) + eps) * (1 + w)); on the first RD dims, with halves
//   x1, x2 and the position's cos/sin: o1 = bf16(bf16(x1 c) + bf16(-x2 s)),
//   o2 = bf16(bf16(x2 c) + bf16(x1 s)). q is written bf16; k and the raw v go to cache row
//   pos + t as fp8(x / sc) with sc = max(amax(x), 1e-6) / 448.
//   attention: query t of head h sees cache rows <= pos + t; scores q . bf16(k8 * ksc) / sqrt(D);
//   online softmax in fp32 (base 2 on the device: maxima and exponents in log2 units) with l
//   summed before the value scale, P = bf16(p * vsc), acc += P v8;
//   splits combined by their maxima; o = bf16(acc / l) * bf16(sigmoid(gate)), bf16 out.
//
// MI355X layout of the split kernel: one workgroup of four waves per (kv head, split); the
// G * M query rows of the kv head (G = HQ / HKV query heads per token) are 16-row MFMA tiles,
// one per wave. Keys stream through LDS 32 at a time: K dequantized to bf16 row-major, V
// converted to bf16 and transposed (d-major) while it is written. Scores are computed transposed,
// S^T = K Q^T (v_mfma_f32_16x16x32_bf16, Q^T stationary in registers), which leaves each lane
// the scores of one query row for 8 keys: exactly the B operand of O^T = V^T P^T once the key
// order inside the 32-key step is permuted the same way on the V^T side. Row maxima and sums
// need two xor shuffles. Each wave keeps O^T for its 16 rows x 256 d in 64 registers.
#include "accept_common.h"

namespace tr {

constexpr int kAttnD = 256;      // head dim
constexpr int kAttnBlk = 32;     // keys per LDS block
constexpr int kAttnMaxM = 8;     // query tokens per chain step
constexpr int kAttnMaxTree = 32; // query tokens (nodes) per draft-tree step: one bit each in a mask word
constexpr int kAttnWaves = 4;
constexpr int kKPitch = kAttnD + 8;     // bf16 elements per K row in LDS
constexpr int kVPitch = kAttnBlk + 4;   // bf16 elements per V^T row (one d) in LDS
constexpr float kFp8Max = 448.f;
constexpr float kLog2e = 1.4426950408889634f;  // scores are kept in log2 units: p = 2^(s - m)
constexpr int kMaxSplit = 256;  // key-range splits of one flash-decoding call
static_assert(kMaxSplit <= kAttnD, "the combine kernel gives each split one thread");

// ------------------------------------------------------------------ fp8 e4m3fn (OCP) helpers

// fp32 -> fp8 e4m3fn bits, round to nearest even; magnitudes past the largest finite value
// (448) saturate to it (the writers keep |x| <= 448 up to rounding).
__device__ __forceinline__ uint32_t f32_to_fp8(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t sign = (u >> 24) & 0x80;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0x1p-6f) {
    code = (uint32_t)__builtin_rintf(a * 512.f);  // subnormal steps of 2^-9; 8 becomes 2^-6
  } else {
    uint32_t v = __float_as_uint(a);
    v += 0x7FFFFu + ((v >> 20) & 1u);            // round the mantissa to 3 bits
    const int e = (int)(v >> 23) - 120;
    const uint32_t m = (v >> 20) & 7;
    code = (e > 15 || (e == 15 && m == 7)) ? 0x7Eu : ((uint32_t)e << 3) | m;
  }
  return sign | code;
}

__device__ __forceinline__ float bf16r_a(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

typedef float f32x2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
// Two fp32 -> packed bf16 (round to nearest even, v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pk_bf16(float x, float y) {
  const bf16x2v r = {(__bf16)x, (__bf16)y};
  return __builtin_bit_cast(uint32_t, r);
}
// fp8 e4m3fn bytes 0,1 (hi = false) or 2,3 (hi = true) of w -> fp32, exact (v_cvt_pk_f32_fp8).
__device__ __forceinline__ f32x2v fp8x2_to_f32(uint32_t w, bool hi) {
  return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true) : __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
}
// Exact fp8 -> bf16 of two values: the fp32 images have zero low halves.
__device__ __forceinline__ uint32_t fp8x2_to_bf16(uint32_t w, bool hi) {
  const f32x2v f = fp8x2_to_f32(w, hi);
  return (__float_as_uint(f.x) >> 16) | (__float_as_uint(f.y) & 0xFFFF0000u);
}
__device__ __forceinline__ float max_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ------------------------------------------------------------------ prep

struct AttnPrepArgs {
  const uint16_t* qkv;   // [M, QKV] bf16
  const uint16_t* qn_w;  // [D] bf16
  const uint16_t* kn_w;  // [D] bf16
  const uint16_t* cos;   // [max_pos, RD] bf16
  const uint16_t* sin;
  const int64_t* pos;
  uint8_t* k_cache;      // [HKV, maxlen, D] fp8
  uint8_t* v_cache;
  float* k_scale;        // [HKV, maxlen]
  float* v_scale;
  uint16_t* q_out;       // [M, HQ, D] bf16
  const int32_t* parent; // [M] draft-tree parents, or null for a chain
  int HQ, HKV, RD, maxlen, ld;
  float eps;
};

// Parent of node t of a draft tree (parent[t] < t; node 0 is the root). A parent outside
// 0..t-1 reads as the root, so every walk up the tree ends within t steps.
__device__ __forceinline__ int attn_tree_parent(const int32_t* parent, int t) {
  const int p = parent[t];
  return (p >= 0 && p < t) ? p : 0;
}

// One wave per (head, token); lane l holds dims 4 l .. 4 l + 3. Token t is written to cache row
// pos + t and roped at position pos + t, or, for node t of a draft tree, at pos + depth(t): the
// position it takes once its root path is committed.
__global__ __launch_bounds__(64) void attn_prep_kernel(AttnPrepArgs a) {
  const int head = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  int dep = t;
  if (a.parent) {
    // the depth by walking the parents held one per lane (one load for the wave, then shuffles:
    // a walk of dependent memory loads waited for each)
    const int pl = lane > 0 && lane < (int)gridDim.y ? attn_tree_parent(a.parent, lane) : 0;
    dep = 0;
    for (int j = t; j > 0 && dep < kAttnMaxTree; ++dep) j = __shfl(pl, j);
  }
  // Positions past the cache's end: the rope table (maxlen rows) is read at the last row and no
  // cache row is written (the split kernel reads at most maxlen rows), so nothing outside the
  // cache is touched whatever the device position holds.
  const int64_t p_raw = *a.pos + t, r_raw = *a.pos + dep;
  const bool in_cache = p_raw >= 0 && p_raw < a.maxlen;
  const int64_t p = in_cache ? p_raw : (p_raw < 0 ? 0 : a.maxlen - 1);
  const int64_t pr = r_raw < 0 ? 0 : (r_raw >= a.maxlen ? a.maxlen - 1 : r_raw);
  const bool isq = head < a.HQ;
  const int j = head - a.HQ;
  const uint16_t* row = a.qkv + (size_t)t * a.ld;
  const uint16_t* src = isq ? row + (size_t)head * 2 * kAttnD : row + (size_t)a.HQ * 2 * kAttnD + (size_t)j * kAttnD;
  const uint16_t* w = isq ? a.qn_w : a.kn_w;
  const int d0 = 4 * lane;
  uint16_t cs_raw[4], sn_raw[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (d0 + i) % (a.RD / 2);
    cs_raw[i] = a.cos[(size_t)pr * a.RD + r];
    sn_raw[i] = a.sin[(size_t)pr * a.RD + r];
  }
  float x[4], wv[4];
  {
    const uint2 xu = *(const uint2*)(src + d0), wu = *(const uint2*)(w + d0);
    x[0] = bf16_bits_to_f32(xu.x & 0xFFFFu);
    x[1] = bf16_bits_to_f32(xu.x >> 16);
    x[2] = bf16_bits_to_f32(xu.y & 0xFFFFu);
    x[3] = bf16_bits_to_f32(xu.y >> 16);
    wv[0] = bf16_bits_to_f32(wu.x & 0xFFFFu);
    wv[1] = bf16_bits_to_f32(wu.x >> 16);
    wv[2] = bf16_bits_to_f32(wu.y & 0xFFFFu);
    wv[3] = bf16_bits_to_f32(wu.y >> 16);
  }
  float ss = x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float inv = 1.f / sqrtf(ss / (float)kAttnD + a.eps);
  float xn[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) xn[i] = bf16r_a(x[i] * inv * (1.f + wv[i]));
  // partial rope on dims < RD: dim r pairs with r + RD / 2 (a lane RD / 8 lanes away). The
  // table entries were loaded with x (in-range indices for every dim, used where d < RD).
  const int half = a.RD / 2;
  float out[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float other = __shfl_xor(xn[i], half / 4);
    const int d = d0 + i;
    out[i] = xn[i];
    if (d < a.RD) {
      const float c = bf16_bits_to_f32(cs_raw[i]), s = bf16_bits_to_f32(sn_raw[i]);
      out[i] = d < half ? bf16r_a(bf16r_a(xn[i] * c) + bf16r_a(-other * s))
                        : bf16r_a(bf16r_a(xn[i] * c) + bf16r_a(other * s));
    }
  }
  if (isq) {
    uint16_t* qo = a.q_out + ((size_t)t * a.HQ + head) * kAttnD + d0;
    uint2 st;
    st.x = (uint32_t)f32_to_bf16_bits(out[0]) | ((uint32_t)f32_to_bf16_bits(out[1]) << 16);
    st.y = (uint32_t)f32_to_bf16_bits(out[2]) | ((uint32_t)f32_to_bf16_bits(out[3]) << 16);
    *(uint2*)qo = st;
    return;
  }
  if (!in_cache) return;
  // key: fp8 with one scale per (head, position)
  float am = fmaxf(fmaxf(fabsf(out[0]), fabsf(out[1])), fmaxf(fabsf(out[2]), fabsf(out[3])));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
  const float sc = fmaxf(am, 1e-6f) / kFp8Max;
  const size_t crow = ((size_t)j * a.maxlen + p);
  uint32_t kb = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) kb |= f32_to_fp8(out[i] / sc) << (8 * i);
  *(uint32_t*)(a.k_cache + crow * kAttnD + d0) = kb;
  // value: raw bf16 from qkv
  const uint2 vu = *(const uint2*)(row + (size_t)a.HQ * 2 * kAttnD + (size_t)(a.HKV + j) * kAttnD + d0);
  const float v[4] = {bf16_bits_to_f32(vu.x & 0xFFFFu), bf16_bits_to_f32(vu.x >> 16), bf16_bits_to_f32(vu.y & 0xFFFFu),
                      bf16_bits_to_f32(vu.y >> 16)};
  float vm = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) vm = fmaxf(vm, __shfl_xor(vm, o));
  const float sv = fmaxf(vm, 1e-6f) / kFp8Max;
  uint32_t vb = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) vb |= f32_to_fp8(v[i] / sv) << (8 * i);
  *(uint32_t*)(a.v_cache + crow * kAttnD + d0) = vb;
  if (lane == 0) {
    a.k_scale[crow] = sc;
    a.v_scale[crow] = sv;
  }
}

// ------------------------------------------------------------------ split (flash-decoding)

struct AttnSplitArgs {
  const uint16_t* q;       // [M, HQ, D] bf16
  const uint8_t* k_cache;  // [HKV, maxlen, D] fp8
  const uint8_t* v_cache;
  const float* k_scale;    // [HKV, maxlen]
  const float* v_scale;
  const int64_t* pos;
  float* m_part;           // [M HQ, NSPLIT]
  float* l_part;
  float* acc_part;         // [M HQ, NSPLIT, D]
  const int32_t* parent;   // [M] draft-tree parents, or null for a chain
  int HQ, HKV, M, maxlen, nsplit;
  float scale;
};

template <bool TREE>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_split_kernel(AttnSplitArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kAttnBlk * kKPitch];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kAttnD * kVPitch];
  __shared__ float ksc[kAttnBlk], vsc[kAttnBlk];
  const int j = blockIdx.x / a.nsplit, s = blockIdx.x % a.nsplit;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int G = a.HQ / a.HKV;
  const int gy = TREE ? (int)blockIdx.y : 0;  // row group (a chain's M * G rows fit one)
  const int rows = G * a.M - 16 * kAttnWaves * gy;  // this workgroup's row group
  const int64_t pos = *a.pos;
  const int64_t L = pos + a.M;
  const int nblk = (int)((L + kAttnBlk - 1) / kAttnBlk);
  const int per = (nblk + a.nsplit - 1) / a.nsplit;
  const int b0 = s * per, b1 = min(b0 + per, nblk);
  const bool computes = 16 * wave < rows;

  // Q^T operand: lane l holds row 16 wave + l % 16, dims 8 (l / 16) + 32 jj .. + 7
  const int row = 16 * wave + (lane & 15);
  const bool rvalid = row < rows;
  const int grow = 16 * kAttnWaves * gy + row;  // row of the kv head: query qi, head g
  const int qi = rvalid ? grow / G : 0;
  const int hq = j * G + (rvalid ? grow % G : 0);
  uint4 qb[8];
#pragma unroll
  for (int jj = 0; jj < 8; ++jj)
    qb[jj] = rvalid ? *(const uint4*)(a.q + ((size_t)qi * a.HQ + hq) * kAttnD + 8 * (lane >> 4) + 32 * jj)
                    : make_uint4(0, 0, 0, 0);
  // The new keys query qi sees: rows pos + i for the bits i of vis -- i <= qi for a chain, the
  // node's ancestors and itself for a tree.
  uint32_t vis = qi >= 31 ? ~0u : (2u << qi) - 1u;
  const int64_t qlimit = pos + qi;  // a chain's last visible row
  if (TREE) {
    // the parents one per lane (one load for the wave), then the walk by shuffles
    const int pl = lane > 0 && lane < a.M ? attn_tree_parent(a.parent, lane) : 0;
    vis = 0;
    int jn = qi;
    for (int d = 0; d < kAttnMaxTree; ++d) {
      vis |= 1u << jn;
      jn = __shfl(pl, jn);  // the root's entry is 0
      if (__all(jn == 0)) break;
    }
    vis |= 1u;  // the root: every node sees it
  }

  f32x4 acc[16];
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_i = -INFINITY, l_i = 0.f;

  // Cache reads go through buffer resources sized to the L live rows: rows past them, and the
  // prefetch past the split's last block, read zeros with no memory access and no branch.
  const int liveL = (int)min(max(L, (int64_t)0), (int64_t)a.maxlen);   // never past the cache
  const auto krs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.k_cache + (size_t)j * a.maxlen * kAttnD), (short)0,
                                                     liveL * kAttnD, 0x00020000);
  const auto vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(a.v_cache + (size_t)j * a.maxlen * kAttnD), (short)0,
                                                     liveL * kAttnD, 0x00020000);
  const auto ksr = __builtin_amdgcn_make_buffer_rsrc((void*)(a.k_scale + (size_t)j * a.maxlen), (short)0, liveL * 4,
                                                     0x00020000);
  const auto vsr = __builtin_amdgcn_make_buffer_rsrc((void*)(a.v_scale + (size_t)j * a.maxlen), (short)0, liveL * 4,
                                                     0x00020000);
  constexpr int kOob = 0x7FFFFFF0;
  // fill roles: K: thread t loads key t / 8, dims 32 (t % 8) .. + 31; V: keys 4 (t % 8) .. + 3,
  // dims 8 (t / 8) .. + 7; scales: threads 0..31 (V) and every 8th thread (K)
  const int fk = tid >> 3, fkd = 32 * (tid & 7);
  const int fv = 4 * (tid & 7), fvd = 8 * (tid >> 3);
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u2 __attribute__((ext_vector_type(2)));
  u4 pk0, pk1;
  u2 pv[4];
  float psk, psv;
  // the cache rows are read once per step: non-temporal, as the GEMM streams its weights
  constexpr int kNt = 2;
  auto fetch = [&](int blk, bool on) {
    const int key0 = blk * kAttnBlk;
    const int kk = key0 + fk;
    pk0 = __builtin_amdgcn_raw_buffer_load_b128(krs, on ? kk * kAttnD + fkd : kOob, 0, kNt);
    pk1 = __builtin_amdgcn_raw_buffer_load_b128(krs, on ? kk * kAttnD + fkd + 16 : kOob, 0, kNt);
    psk = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ksr, on ? kk * 4 : kOob, 0, kNt));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      pv[i] = __builtin_amdgcn_raw_buffer_load_b64(vrs, on ? (key0 + fv + i) * kAttnD + fvd : kOob, 0, kNt);
    psv = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(vsr, on && tid < kAttnBlk ? (key0 + tid) * 4 : kOob, 0, kNt));
  };
  fetch(b0, b0 < b1);
  for (int blk = b0; blk < b1; ++blk) {
    const int64_t key0 = (int64_t)blk * kAttnBlk;
    __syncthreads();  // the previous block's LDS reads are done
    {
      const uint32_t kw[8] = {pk0.x, pk0.y, pk0.z, pk0.w, pk1.x, pk1.y, pk1.z, pk1.w};
      const float sck = psk;
      uint16_t* dst = Ks + fk * kKPitch + fkd;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        uint32_t o[4];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const f32x2v f = fp8x2_to_f32(kw[2 * q4 + h / 2], h & 1);
          o[h] = pk_bf16(f.x * sck, f.y * sck);
        }
        *(uint4*)(dst + 8 * q4) = make_uint4(o[0], o[1], o[2], o[3]);
      }
      if ((tid & 7) == 0) ksc[fk] = sck;
    }
    {
      // 4 keys x 8 dims -> 8 rows of V^T (4 keys each): byte e of key i is pv[i] byte e. One
      // v_perm_b32 gathers byte e of two keys, one scaled conversion (scale 1: exact) makes the
      // bf16 pair.
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t sel = 0x0C0C0000u | ((4u + (e & 3)) << 8) | (uint32_t)(e & 3);  // b0 = lo[e], b1 = hi[e]
        const uint32_t w01 = __builtin_amdgcn_perm(e < 4 ? pv[1].x : pv[1].y, e < 4 ? pv[0].x : pv[0].y, sel);
        const uint32_t w23 = __builtin_amdgcn_perm(e < 4 ? pv[3].x : pv[3].y, e < 4 ? pv[2].x : pv[2].y, sel);
        uint2 o;
        o.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w01, 1.f, false));
        o.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w23, 1.f, false));
        *(uint2*)(Vt + (fvd + e) * kVPitch + fv) = o;
      }
      if (tid < kAttnBlk) vsc[tid] = psv;
    }
    fetch(blk + 1, blk + 1 < b1);  // the next block's loads run under this block's compute
    __syncthreads();
    if (!computes) continue;
    // S^T = K Q^T for the block's two 16-key tiles: lane gets keys 16 kt + 4 (l / 16) + r, row l % 16
    f32x4 st[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* kr = Ks + (16 * kt + (lane & 15)) * kKPitch + 8 * (lane >> 4);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const uint4 kv = *(const uint4*)(kr + 32 * jj);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kv), __builtin_bit_cast(bf16x8, qb[jj]),
                                                    c, 0, 0, 0);
      }
      st[kt] = c;
    }
    // mask, online softmax (this lane: one row, 8 keys), in log2 units: p = 2^(s - m) by
    // v_exp_f32 (one instruction where expf takes a range reduction)
    const float sl2 = a.scale * kLog2e;
    float sc[8];
    float mx = -INFINITY;
    // a block of committed rows only (all before pos) needs no mask; in the others key rel =
    // kidx - pos < M selects a bit of vis when >= 0
    const bool committed = TREE && key0 + kAttnBlk <= pos;  // uniform
    const int rel0 = TREE ? (int)(key0 - pos) + 4 * (lane >> 4) : 0;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int rel = rel0 + 16 * kt + r;
        const bool allowed =
            TREE ? rvalid && (committed || (rel < a.M && (rel < 0 || ((vis >> rel) & 1u))))
                 : rvalid && key0 + 16 * kt + 4 * (lane >> 4) + r < L && key0 + 16 * kt + 4 * (lane >> 4) + r <= qlimit;
        const float v = allowed ? st[kt][r] * sl2 : -INFINITY;
        sc[4 * kt + r] = v;
        mx = fmaxf(mx, v);
      }
    mx = max_x32(max_x16(mx));
    // Lazy rescale: the rows move to their new maxima (and O^T, l are scaled) only when some row
    // of the wave gains more than kLazyMax (log2 units) over its running max; otherwise the block
    // is summed against the running max, so p <= 2^kLazyMax. m, l and O^T stay consistent.
    constexpr float kLazyMax = 8.f;
    if (__ballot(mx > m_i + kLazyMax)) {  // uniform; a first finite maximum always counts
      const float m_new = fmaxf(m_i, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_i - (m_new == -INFINITY ? 0.f : m_new));
      m_i = m_new;
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < 16; ++dt) acc[dt] = acc[dt] * alpha;
    }
    const float m_safe = m_i == -INFINITY ? 0.f : m_i;
    float psum = 0.f;
    uint32_t pb[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const float p0 = __builtin_amdgcn_exp2f(sc[i] - m_safe), p1 = __builtin_amdgcn_exp2f(sc[i + 1] - m_safe);
      psum += p0 + p1;
      const int k0 = 16 * (i / 4) + 4 * (lane >> 4) + (i & 3);
      pb[i / 2] = pk_bf16(p0 * vsc[k0], p1 * vsc[k0 + 1]);
    }
    psum = sum_x32(sum_x16(psum));
    l_i += psum;
    // O^T += V^T P^T: k-index 8 (l / 16) + i <-> key 4 (l / 16) + i (i < 4), 16 + 4 (l / 16) + i - 4
    const bf16x8 pB = __builtin_bit_cast(bf16x8, make_uint4(pb[0], pb[1], pb[2], pb[3]));
    const int vk = 4 * (lane >> 4);
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) {
      const uint16_t* vr = Vt + (16 * dt + (lane & 15)) * kVPitch;
      const uint2 lo = *(const uint2*)(vr + vk), hi = *(const uint2*)(vr + 16 + vk);
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y)),
                                                        pB, acc[dt], 0, 0, 0);
    }
  }
  if (!computes || !rvalid) return;
  // lanes with l / 16 == 0 .. 3 hold d = 16 dt + 4 (l / 16) + r of row l % 16
  const size_t h = (size_t)qi * a.HQ + hq;
  if (lane < 16) {
    a.m_part[h * a.nsplit + s] = m_i;
    a.l_part[h * a.nsplit + s] = l_i;
  }
  float* ap = a.acc_part + (h * a.nsplit + s) * kAttnD + 4 * (lane >> 4);
#pragma unroll
  for (int dt = 0; dt < 16; ++dt) *(float4*)(ap + 16 * dt) = make_float4(acc[dt][0], acc[dt][1], acc[dt][2], acc[dt][3]);
}

// ------------------------------------------------------------------ reduce + output gate

struct AttnReduceArgs {
  const float* m_part;
  const float* l_part;
  const float* acc_part;
  const uint16_t* qkv;  // [M, QKV] for the gates
  uint16_t* out;        // [M, HQ D]
  int HQ, nsplit, ld;
};

// One workgroup of D threads per (token, query head). Every load is issued up front: the split
// accumulators of this thread's dimension in batches of 64 (clamped indices past nsplit, weight
// 0), one split's (m, l) per thread, and the gate; the split maximum and the weighted total are
// block reductions.
__global__ __launch_bounds__(kAttnD) void attn_reduce_kernel(AttnReduceArgs a) {
  constexpr int kB = 64;
  __shared__ float wsh[kMaxSplit], red[kAttnD / 64];
  const int h = blockIdx.x, d = threadIdx.x, lane = d & 63, wave = d >> 6;
  const int ns = a.nsplit;
  const int t = h / a.HQ, hh = h % a.HQ;
  const uint16_t graw = a.qkv[(size_t)t * a.ld + (size_t)hh * 2 * kAttnD + kAttnD + d];
  const float* ap = a.acc_part + (size_t)h * ns * kAttnD + d;
  float v[kB];
#pragma unroll
  for (int i = 0; i < kB; ++i) v[i] = ap[(size_t)min(i, ns - 1) * kAttnD];
  const int sc = min(d, ns - 1);
  const float m_s = a.m_part[(size_t)h * ns + sc], l_s = a.l_part[(size_t)h * ns + sc];
  const bool mine = d < ns;  // ns <= kMaxSplit == kAttnD
  // maximum over the splits
  float mm = mine ? m_s : -INFINITY;
  mm = fmaxf(mm, __shfl_xor(mm, 32));
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) mm = fmaxf(mm, __shfl_xor(mm, o));
  if (lane == 0) red[wave] = mm;
  __syncthreads();
  mm = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float w = mine && m_s != -INFINITY ? __builtin_amdgcn_exp2f(m_s - mm) : 0.f;  // maxima in log2 units
  if (mine) wsh[d] = w;
  // total weight sum_s w_s l_s
  float lt = sum_wave(w * l_s);
  __syncthreads();  // red[] reads done, wsh[] written
  if (lane == 0) red[wave] = lt;
  __syncthreads();
  lt = ((red[0] + red[1]) + red[2]) + red[3];
  float o = 0.f;
#pragma unroll
  for (int i = 0; i < kB; ++i)
    if (i < ns) o += wsh[i] * v[i];
  for (int s0 = kB; s0 < ns; s0 += kB) {  // nsplit > 64: further batches
#pragma unroll
    for (int i = 0; i < kB; ++i) v[i] = ap[(size_t)min(s0 + i, ns - 1) * kAttnD];
#pragma unroll
    for (int i = 0; i < kB; ++i)
      if (s0 + i < ns) o += wsh[s0 + i] * v[i];
  }
  o = bf16r_a(o / lt);
  const float gate = bf16_bits_to_f32(graw);
  const float g = bf16r_a(1.f / (1.f + expf(-gate)));
  a.out[(size_t)h * kAttnD + d] = f32_to_bf16_bits(o * g);
}

}  // namespace tr

using namespace tr;

extern "C" {

size_t tr_attn_workspace_bytes(int M, int HQ, int nsplit) {
  if (M < 1 || M > kAttnMaxTree || HQ < 1 || nsplit < 1) return 0;
  const size_t rows = (size_t)M * HQ * nsplit;
  return rows * (2 + kAttnD) * sizeof(float);
}

}  // extern "C"

namespace {

int attn_prep_launch(const void* qkv, int ld, const void* q_norm_w, const void* k_norm_w, const void* cos,
                     const void* sin, int rotary_dim, const int64_t* pos, void* k_cache, void* v_cache, float* k_scale,
                     float* v_scale, int maxlen, void* q_out, int M, int HQ, int HKV, int D, float eps,
                     const int32_t* parent, void* stream) {
  // rotary_dim: a power of two (its two halves are then an xor-shuffle apart) in [8, D]
  if (D != kAttnD || HQ < 1 || HKV < 1 || HQ % HKV || (rotary_dim & (rotary_dim - 1)) || rotary_dim < 8 ||
      rotary_dim > D || maxlen < M)
    return TR_ERR_SHAPE;
  if (!qkv || !q_norm_w || !k_norm_w || !cos || !sin || !pos || !k_cache || !v_cache || !k_scale || !v_scale || !q_out)
    return TR_ERR_ARG;
  if (ld < 2 * HQ * D + 2 * HKV * D) return TR_ERR_ARG;
  AttnPrepArgs a;
  a.qkv = (const uint16_t*)qkv;
  a.qn_w = (const uint16_t*)q_norm_w;
  a.kn_w = (const uint16_t*)k_norm_w;
  a.cos = (const uint16_t*)cos;
  a.sin = (const uint16_t*)sin;
  a.pos = pos;
  a.k_cache = (uint8_t*)k_cache;
  a.v_cache = (uint8_t*)v_cache;
  a.k_scale = k_scale;
  a.v_scale = v_scale;
  a.q_out = (uint16_t*)q_out;
  a.parent = parent;
  a.HQ = HQ;
  a.HKV = HKV;
  a.RD = rotary_dim;
  a.maxlen = maxlen;
  a.ld = ld;
  a.eps = eps;
  hipLaunchKernelGGL(attn_prep_kernel, dim3(HQ + HKV, M), dim3(64), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int attn_decode_launch(const void* q, const void* qkv, int ld, const void* k_cache, const void* v_cache,
                       const float* k_scale, const float* v_scale, int maxlen, const int64_t* pos, void* out,
                       void* workspace, size_t workspace_bytes, int M, int HQ, int HKV, int D, int nsplit,
                       const int32_t* parent, void* stream) {
  if (D != kAttnD || HQ < 1 || HKV < 1 || HQ % HKV || nsplit < 1 || nsplit > kMaxSplit || maxlen < M)
    return TR_ERR_SHAPE;
  if (!q || !qkv || !k_cache || !v_cache || !k_scale || !v_scale || !pos || !out || !workspace) return TR_ERR_ARG;
  if (ld < 2 * HQ * D + 2 * HKV * D || workspace_bytes < tr_attn_workspace_bytes(M, HQ, nsplit)) return TR_ERR_ARG;
  const size_t rows = (size_t)M * HQ * nsplit;
  AttnSplitArgs s;
  s.q = (const uint16_t*)q;
  s.k_cache = (const uint8_t*)k_cache;
  s.v_cache = (const uint8_t*)v_cache;
  s.k_scale = k_scale;
  s.v_scale = v_scale;
  s.pos = pos;
  s.m_part = (float*)workspace;
  s.l_part = s.m_part + rows;
  s.acc_part = s.l_part + rows;
  s.parent = parent;
  s.HQ = HQ;
  s.HKV = HKV;
  s.M = M;
  s.maxlen = maxlen;
  s.nsplit = nsplit;
  s.scale = 1.f / sqrtf((float)D);
  // the G M query rows of a kv head in groups of 64 (one 16-row tile per wave)
  const int groups = ((HQ / HKV) * M + 16 * kAttnWaves - 1) / (16 * kAttnWaves);
  if (parent)
    hipLaunchKernelGGL(attn_split_kernel<true>, dim3(HKV * nsplit, groups), dim3(64 * kAttnWaves), 0,
                       (hipStream_t)stream, s);
  else
    hipLaunchKernelGGL(attn_split_kernel<false>, dim3(HKV * nsplit, groups), dim3(64 * kAttnWaves), 0,
                       (hipStream_t)stream, s);
  if (hipGetLastError() != hipSuccess) return TR_ERR_LAUNCH;
  AttnReduceArgs r;
  r.m_part = s.m_part;
  r.l_part = s.l_part;
  r.acc_part = s.acc_part;
  r.qkv = (const uint16_t*)qkv;
  r.out = (uint16_t*)out;
  r.HQ = HQ;
  r.nsplit = nsplit;
  r.ld = ld;
  hipLaunchKernelGGL(attn_reduce_kernel, dim3(M * HQ), dim3(kAttnD), 0, (hipStream_t)stream, r);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int tr_attn_prep(const void* qkv, int ld, const void* q_norm_w, const void* k_norm_w, const void* cos,
                 const void* sin, int rotary_dim, const int64_t* pos, void* k_cache, void* v_cache, float* k_scale,
                 float* v_scale, int maxlen, void* q_out, int M, int HQ, int HKV, int D, float eps, void* stream) {
  if (M == 0) return TR_OK;
  if (M < 0 || M > kAttnMaxM) return TR_ERR_SHAPE;
  return attn_prep_launch(qkv, ld, q_norm_w, k_norm_w, cos, sin, rotary_dim, pos, k_cache, v_cache, k_scale, v_scale,
                          maxlen, q_out, M, HQ, HKV, D, eps, nullptr, stream);
}

int tr_attn_decode(const void* q, const void* qkv, int ld, const void* k_cache, const void* v_cache,
                   const float* k_scale, const float* v_scale, int maxlen, const int64_t* pos, void* out,
                   void* workspace, size_t workspace_bytes, int M, int HQ, int HKV, int D, int nsplit, void* stream) {
  if (M == 0) return TR_OK;
  // a chain's query rows of one kv head fit one workgroup's four 16-row tiles
  if (M < 0 || M > kAttnMaxM || HQ < 1 || HKV < 1 || (HQ / HKV) * M > 16 * kAttnWaves) return TR_ERR_SHAPE;
  return attn_decode_launch(q, qkv, ld, k_cache, v_cache, k_scale, v_scale, maxlen, pos, out, workspace,
                            workspace_bytes, M, HQ, HKV, D, nsplit, nullptr, stream);
}

int tr_attn_prep_tree(const void* qkv, int ld, const void* q_norm_w, const void* k_norm_w, const void* cos,
                      const void* sin, int rotary_dim, const int64_t* pos, const int32_t* parent, void* k_cache,
                      void* v_cache, float* k_scale, float* v_scale, int maxlen, void* q_out, int M, int HQ, int HKV,
                      int D, float eps, void* stream) {
  if (M == 0) return TR_OK;
  if (M < 0 || M > kAttnMaxTree) return TR_ERR_SHAPE;
  if (!parent) return TR_ERR_ARG;
  return attn_prep_launch(qkv, ld, q_norm_w, k_norm_w, cos, sin, rotary_dim, pos, k_cache, v_cache, k_scale, v_scale,
                          maxlen, q_out, M, HQ, HKV, D, eps, parent, stream);
}

int tr_attn_decode_tree(const void* q, const void* qkv, int ld, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale, int maxlen, const int64_t* pos,
                        const int32_t* parent, void* out, void* workspace, size_t workspace_bytes, int M, int HQ,
                        int HKV, int D, int nsplit, void* stream) {
  if (M == 0) return TR_OK;
  if (M < 0 || M > kAttnMaxTree) return TR_ERR_SHAPE;
  if (!parent) return TR_ERR_ARG;
  return attn_decode_launch(q, qkv, ld, k_cache, v_cache, k_scale, v_scale, maxlen, pos, out, workspace,
                            workspace_bytes, M, HQ, HKV, D, nsplit, parent, stream);
}

}  // extern "C"
