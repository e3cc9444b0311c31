// M-token gated-delta-rule (GDN) verify step for gfx950: causal conv over the ring, b/a gates,
// the recurrence with a state snapshot after every token, and the gated RMSNorm output.
//
// Follows the reference's fused decode kernel (tokenrush/fused.py:94-210, _gdn_step_fused_kernel
// and _gated_norm_kernel) and its eager ops (tokenrush/ops.py:10-30 gated_rmsnorm, :99-113
// conv_step, :150-161 gdn_step_reference). For token t = 0..M-1 at position pos + t and value
// head hv (key head ih = hv / (HV / H)):
//
//   conv:  c = bf16(silu(bf16(s0 w0 + s1 w1 + s2 w2 + x_t w3)))  per conv channel, where
//          s0..s2 are the channel's inputs at positions pos + t - 3 .. pos + t - 1 (the ring for
//          positions before pos, this step's rows after) and x_t = qkvz[t, ch]; the ring column
//          (pos + t) % R receives x_t.
//   gates: b, a = bf16(x_t . ba_w[hv]), bf16(x_t . ba_w[HV + hv])  (fp32 accumulate)
//          beta = bf16(sigmoid(b)), g = A[hv] * softplus(a + dt_bias[hv])
//   q = c_q / sqrt(|c_q|^2 + 1e-6) * K^-1/2,  k = c_k / sqrt(|c_k|^2 + 1e-6)
//   S = S * exp(g);  S += k (beta (v - k^T S))^T;  snapshot slot t <- S;  o = q^T S
//   y = bf16(bf16(w * bf16(o_b * rsqrt(mean(o_b^2) + eps))) * silu(z)),  o_b = bf16(o)
//
// The committed state is read from slot *slot of rec; the state after token t is written to
// slot t, so the accept can commit any prefix by naming its slot (tokenrush/state.py:30-39).
//
// Layout and work split (MI355X): one 64-lane wave per (value head, 32-column block of V), so
// a layer's 48 x 4 = 192 workgroups spread the 64 KB-per-head state over the CUs. Lane
// (vq = lane % 8, kg = lane / 8) holds S[16 kg .. 16 kg + 15][4 vq .. 4 vq + 3] of its block in
// registers for all M tokens; its snapshot stores are 16-byte vectors, 8 lanes per 128-byte row
// segment. Sums over k combine each lane's 16 rows, then lanes kg = 0..7 by xor shuffles. The
// conv outputs of all M tokens (128 q, 128 k and 32 v channels) are computed up front into LDS.
// The gated norm needs the whole head: the four column blocks store bf16 o to a workspace with
// agent-scope stores, and the last of them to arrive normalizes the head for every token.
#include "accept_common.h"

namespace tr {

constexpr int kGdnK = 128;   // key head dim
constexpr int kGdnV = 128;   // value head dim
constexpr int kGdnBV = 32;   // value columns per workgroup
constexpr int kGdnNVB = kGdnV / kGdnBV;
constexpr int kGdnMaxM = 8;  // tokens per step (the reference's MP, fused.py:150)

struct GdnArgs {
  const uint16_t* qkvz;    // [M, ld] bf16: q | k | v | z
  const uint16_t* x;       // [M, hidden] bf16, the layer input (b/a gates)
  const uint16_t* ba_w;    // [2 HV, hidden] bf16
  uint16_t* ring;          // [conv_dim, R] bf16
  const uint16_t* conv_w;  // [conv_dim, 4] bf16
  const float* A;          // [HV]
  const float* dt_bias;    // [HV]
  float* rec;              // slot s: rec + s * slot_stride, [HV, K, V] fp32
  const int64_t* slot;     // [1] committed slot
  const int64_t* pos;      // [1] position of token 0
  const uint16_t* norm_w;  // [V] bf16
  uint16_t* y;             // [M, HV V] bf16
  float* o_ws;             // [M, HV V] fp32 (bf16 values), workspace
  int* cnt;                // [HV] arrival counters, one per 128-byte line, zero between calls
  long slot_stride;        // floats
  int ld, hidden, M, H, HV, R;
  float eps, scale;
};

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Sum over the 8 lanes that share lane % 8 (kg = 0..7), in a fixed order for every lane.
__device__ __forceinline__ float kg_sum(float v) {
  v += __shfl_xor(v, 8);
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : logf(1.f + expf(x)); }

__global__ __launch_bounds__(64) void gdn_step_kernel(GdnArgs a) {
  __shared__ float cq[kGdnMaxM][kGdnK], ck[kGdnMaxM][kGdnK], cv[kGdnMaxM][kGdnBV];
  __shared__ int last;
  const int lane = threadIdx.x;
  const int hv = blockIdx.x / kGdnNVB, vb = blockIdx.x % kGdnNVB;
  const int ih = hv / (a.HV / a.H);
  const int M = a.M;
  const int QK = a.H * kGdnK, VAL = a.HV * kGdnV;
  const int64_t pos = *a.pos;
  const int64_t slot = *a.slot;
  const int vq = lane & 7, kg = lane >> 3;
  const int v0 = vb * kGdnBV + 4 * vq;  // this lane's first column within the head

  // Committed state tile, loaded first: everything below overlaps its latency.
  float4 S[16];
  {
    const float* src = a.rec + slot * a.slot_stride + (size_t)hv * kGdnK * kGdnV + v0;
#pragma unroll
    for (int j = 0; j < 16; ++j) S[j] = *(const float4*)(src + (size_t)(16 * kg + j) * kGdnV);
  }

  // b and a gates of every token: per-lane partial dot products over hidden, then a wave sum.
  float bs[kGdnMaxM], as[kGdnMaxM];
#pragma unroll
  for (int t = 0; t < kGdnMaxM; ++t) bs[t] = as[t] = 0.f;
  {
    const uint16_t* wb = a.ba_w + (size_t)hv * a.hidden;
    const uint16_t* wa = a.ba_w + (size_t)(a.HV + hv) * a.hidden;
    for (int e = 8 * lane; e < a.hidden; e += 8 * 64) {
      const uint4 ub = *(const uint4*)(wb + e), ua = *(const uint4*)(wa + e);
      const uint32_t wbw[4] = {ub.x, ub.y, ub.z, ub.w}, waw[4] = {ua.x, ua.y, ua.z, ua.w};
#pragma unroll
      for (int t = 0; t < kGdnMaxM; ++t) {
        if (t < M) {
          const uint4 ux = *(const uint4*)(a.x + (size_t)t * a.hidden + e);
          const uint32_t xw[4] = {ux.x, ux.y, ux.z, ux.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x0 = bf16_bits_to_f32(xw[i] & 0xFFFFu), x1 = bf16_bits_to_f32(xw[i] >> 16);
            bs[t] += x0 * bf16_bits_to_f32(wbw[i] & 0xFFFFu) + x1 * bf16_bits_to_f32(wbw[i] >> 16);
            as[t] += x0 * bf16_bits_to_f32(waw[i] & 0xFFFFu) + x1 * bf16_bits_to_f32(waw[i] >> 16);
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kGdnMaxM; ++t) {
      bs[t] = bf16r(wave_sum_f(bs[t]));
      as[t] = bf16r(wave_sum_f(as[t]));
    }
  }

  // Causal conv + silu of this workgroup's 288 channels for all M tokens, into LDS. The ring
  // column of position p is p % R; positions pos..pos+M-1 are this step's qkvz rows. The q/k
  // channels of a key head are shared by HV / H value heads and four column blocks: only the
  // first of them writes those ring columns (identical values; one writer keeps it race-free).
  const bool qk_owner = (hv % (a.HV / a.H)) == 0 && vb == 0;
  for (int idx = lane; idx < 2 * kGdnK + kGdnBV; idx += 64) {
    int ch;
    float* dst;
    bool own;
    if (idx < kGdnK) {
      ch = ih * kGdnK + idx;
      dst = &cq[0][idx];
      own = qk_owner;
    } else if (idx < 2 * kGdnK) {
      ch = QK + ih * kGdnK + (idx - kGdnK);
      dst = &ck[0][idx - kGdnK];
      own = qk_owner;
    } else {
      ch = 2 * QK + hv * kGdnV + vb * kGdnBV + (idx - 2 * kGdnK);
      dst = &cv[0][idx - 2 * kGdnK];
      own = true;
    }
    const int stride = idx < 2 * kGdnK ? kGdnK : kGdnBV;  // LDS row pitch of dst
    const uint2 wu = *(const uint2*)(a.conv_w + (size_t)ch * 4);
    const float w0 = bf16_bits_to_f32(wu.x & 0xFFFFu), w1 = bf16_bits_to_f32(wu.x >> 16);
    const float w2 = bf16_bits_to_f32(wu.y & 0xFFFFu), w3 = bf16_bits_to_f32(wu.y >> 16);
    float win[kGdnMaxM + 3];
    const uint16_t* rrow = a.ring + (size_t)ch * a.R;
#pragma unroll
    for (int j = 0; j < 3; ++j) win[j] = bf16_bits_to_f32(rrow[(int)((pos + j - 3 + 4 * (int64_t)a.R) % a.R)]);
#pragma unroll
    for (int t = 0; t < kGdnMaxM; ++t) win[t + 3] = t < M ? bf16_bits_to_f32(a.qkvz[(size_t)t * a.ld + ch]) : 0.f;
#pragma unroll
    for (int t = 0; t < kGdnMaxM; ++t) {
      if (t < M) {
        float yv = win[t] * w0;
        yv = yv + win[t + 1] * w1;
        yv = yv + win[t + 2] * w2;
        yv = yv + win[t + 3] * w3;
        yv = bf16r(yv);
        dst[t * stride] = bf16r(yv / (1.f + expf(-yv)));
      }
    }
    if (own) {
      uint16_t* wrow = a.ring + (size_t)ch * a.R;
      for (int t = 0; t < M; ++t) wrow[(int)((pos + t) % a.R)] = a.qkvz[(size_t)t * a.ld + ch];
    }
  }
  __syncthreads();

  const float Ah = a.A[hv], dtb = a.dt_bias[hv];
  float* const obase = a.o_ws + (size_t)hv * kGdnV + v0;
  for (int t = 0; t < M; ++t) {
    // L2 norms of this token's q and k (all 128 channels), then this lane's 16 rows of each
    float sq = cq[t][lane] * cq[t][lane] + cq[t][lane + 64] * cq[t][lane + 64];
    float sk = ck[t][lane] * ck[t][lane] + ck[t][lane + 64] * ck[t][lane + 64];
    const float nq = sqrtf(wave_sum_f(sq) + 1e-6f), nk = sqrtf(wave_sum_f(sk) + 1e-6f);
    float qk[16], kk[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      qk[j] = cq[t][16 * kg + j] / nq * a.scale;
      kk[j] = ck[t][16 * kg + j] / nk;
    }
    const float beta = bf16r(1.f / (1.f + expf(-bs[t])));
    const float eg = expf(Ah * softplus_f(as[t] + dtb));
    // decay, then the delta-rule correction along k
    float4 kv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      S[j].x *= eg;
      S[j].y *= eg;
      S[j].z *= eg;
      S[j].w *= eg;
      kv.x += S[j].x * kk[j];
      kv.y += S[j].y * kk[j];
      kv.z += S[j].z * kk[j];
      kv.w += S[j].w * kk[j];
    }
    kv.x = kg_sum(kv.x);
    kv.y = kg_sum(kv.y);
    kv.z = kg_sum(kv.z);
    kv.w = kg_sum(kv.w);
    const float* vt = &cv[t][4 * vq];
    float4 dv;
    dv.x = beta * (vt[0] - kv.x);
    dv.y = beta * (vt[1] - kv.y);
    dv.z = beta * (vt[2] - kv.z);
    dv.w = beta * (vt[3] - kv.w);
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    float* dst = a.rec + (size_t)t * a.slot_stride + (size_t)hv * kGdnK * kGdnV + v0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      S[j].x += kk[j] * dv.x;
      S[j].y += kk[j] * dv.y;
      S[j].z += kk[j] * dv.z;
      S[j].w += kk[j] * dv.w;
      *(float4*)(dst + (size_t)(16 * kg + j) * kGdnV) = S[j];
      o.x += S[j].x * qk[j];
      o.y += S[j].y * qk[j];
      o.z += S[j].z * qk[j];
      o.w += S[j].w * qk[j];
    }
    o.x = kg_sum(o.x);
    o.y = kg_sum(o.y);
    o.z = kg_sum(o.z);
    o.w = kg_sum(o.w);
    if (kg == 0) {
      float* op = obase + (size_t)t * VAL;
      ws_st(op + 0, bf16r(o.x));
      ws_st(op + 1, bf16r(o.y));
      ws_st(op + 2, bf16r(o.z));
      ws_st(op + 3, bf16r(o.w));
    }
  }

  // The last of the head's column blocks applies the gated norm to all V columns, every token.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (lane == 0) {
    int* c = a.cnt + hv * 32;
    const int old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == kGdnNVB - 1;
    if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  const int Z = 2 * QK + VAL;
  for (int t = 0; t < M; ++t) {
    const float* op = a.o_ws + (size_t)t * VAL + (size_t)hv * kGdnV;
    const float o0 = ws_ld(op + lane), o1 = ws_ld(op + lane + 64);
    const float var = wave_sum_f(o0 * o0 + o1 * o1) / (float)kGdnV;
    const float r = 1.f / sqrtf(var + a.eps);
    const uint16_t* zr = a.qkvz + (size_t)t * a.ld + Z + (size_t)hv * kGdnV;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int v = lane + 64 * h;
      const float ob = h ? o1 : o0;
      const float n = bf16r(bf16r(ob * r) * bf16_bits_to_f32(a.norm_w[v]));
      const float z = bf16_bits_to_f32(zr[v]);
      a.y[(size_t)t * VAL + (size_t)hv * kGdnV + v] = f32_to_bf16_bits(n * (z / (1.f + expf(-z))));
    }
  }
}

}  // namespace tr

using namespace tr;

extern "C" {

size_t tr_gdn_workspace_bytes(int M, int HV) {
  if (M < 1 || M > kGdnMaxM || HV < 1) return 0;
  return (size_t)HV * 32 * sizeof(int) + (size_t)M * HV * kGdnV * sizeof(float);
}

int tr_gdn_step(const void* qkvz, int ld, const void* x, const void* ba_w, void* ring, const void* conv_w,
                const float* A, const float* dt_bias, float* rec, long slot_stride, const int64_t* slot,
                const void* norm_w, const int64_t* pos, void* y, void* workspace, size_t workspace_bytes, int M,
                int H, int HV, int K, int V, int hidden, int R, float eps, void* stream) {
  if (M == 0) return TR_OK;
  if (M < 0 || M > kGdnMaxM || K != kGdnK || V != kGdnV || H < 1 || HV < H || HV % H || hidden < 8 ||
      hidden % 8 || R < M + 3)
    return TR_ERR_SHAPE;
  if (!qkvz || !x || !ba_w || !ring || !conv_w || !A || !dt_bias || !rec || !slot || !norm_w || !pos || !y ||
      !workspace)
    return TR_ERR_ARG;
  if (ld < 2 * H * K + 2 * HV * V || slot_stride < (long)HV * K * V) return TR_ERR_ARG;
  if (workspace_bytes < tr_gdn_workspace_bytes(M, HV)) return TR_ERR_ARG;
  GdnArgs a;
  a.qkvz = (const uint16_t*)qkvz;
  a.x = (const uint16_t*)x;
  a.ba_w = (const uint16_t*)ba_w;
  a.ring = (uint16_t*)ring;
  a.conv_w = (const uint16_t*)conv_w;
  a.A = A;
  a.dt_bias = dt_bias;
  a.rec = rec;
  a.slot = slot;
  a.pos = pos;
  a.norm_w = (const uint16_t*)norm_w;
  a.y = (uint16_t*)y;
  a.cnt = (int*)workspace;
  a.o_ws = (float*)((char*)workspace + (size_t)HV * 32 * sizeof(int));
  a.slot_stride = slot_stride;
  a.ld = ld;
  a.hidden = hidden;
  a.M = M;
  a.H = H;
  a.HV = HV;
  a.R = R;
  a.eps = eps;
  a.scale = 1.f / sqrtf((float)K);
  hipLaunchKernelGGL(gdn_step_kernel, dim3(HV * kGdnNVB), dim3(64), 0, (hipStream_t)stream, a);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"
