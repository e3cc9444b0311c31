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
// Two launches on MI355X:
//   gdn_prep_kernel does the work every column block of a head shares, once: the conv of all
//   channels (one thread per channel, a workgroup per 8 tokens, 4 in trees over 8 nodes; the ring update),
//   the L2 normalisation of q and k (a 256-channel workgroup holds two whole heads), and the gate dot products
//   (one workgroup per gate row and group of 8 tokens, the four waves splitting the hidden dim).
//   gdn_step_kernel runs the recurrence, one workgroup of four waves per (value head, 16-column
//   block): 48 x 8 = 384 workgroups, so the M x 64 KB-per-head snapshot stores -- the kernel's
//   cost -- spread over every CU. Wave w holds rows 32 w .. 32 w + 31 of the block's [128 x 16]
//   state tile; lane (vq = l % 8, kg = l / 8) holds rows 32 w + 4 kg .. + 3, columns 2 vq, 2 vq + 1,
//   in registers for all M tokens, and its snapshot stores are 8-byte vectors, 8 lanes per
//   64-byte row segment. Sums over k: a lane's 4 rows, the wave's 8 row groups (DPP / permlane
//   steps) and the 4 waves (LDS, fixed order), once per token for both o_t and kv_{t+1}.
//   The gated norm needs the whole head: the four blocks store bf16 o with agent-scope stores,
//   and the last of them to arrive normalizes the head for every token.
//
// Draft trees (tr_gdn_tree_step, up to 32 nodes, parent[t] < t): node t is the last token of a
// chain over its root path. The conv window is the node's three nearest ancestors (the ring's
// committed columns where the path is shorter); the ring is not written, the nodes' inputs go to
// node_in and tr_gdn_tree_commit writes the accepted path's into the ring. In the recurrence a
// node whose parent is not the previous node continues from the parent's snapshot, loaded during
// the previous node's work, so every node still costs one cross-wave exchange.
#include "accept_common.h"

namespace tr {

constexpr int kGdnK = 128;   // key head dim
constexpr int kGdnV = 128;   // value head dim
constexpr int kGdnBV = 16;   // value columns per step workgroup: 2 per lane (8 column pairs x 8 row groups)
constexpr int kGdnNVB = kGdnV / kGdnBV;
constexpr int kGdnMaxM = 8;  // tokens per chain step (the reference's MP, fused.py:150)
constexpr int kGdnMaxTree = 32;  // nodes per draft-tree step
// tokens per conv workgroup of the prep: all of a chain step's, 4 of a larger tree's
template <int MAXM> constexpr int gdn_tg() { return MAXM <= 8 ? 8 : 4; }
constexpr int kGdnThreads = 256;
static_assert(kGdnBV == 16, "the step kernel's lane layout: 8 column pairs");

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
  float* o_ws;             // [M, HV V] fp32 (bf16 values), workspace: head outputs for the norm
  int* cnt;                // [HV] arrival counters, one per 128-byte line, zero between calls
  float* qk;               // [M, 2 H K] fp32, workspace: normalised q (times K^-1/2) | k
  uint16_t* vconv;         // [M, HV V] bf16, workspace: conv + silu of the v channels
  float* gates;            // [M, 2 HV] fp32 (bf16 values), workspace: b | a
  const int32_t* parent;   // [M] draft-tree parents, or null for a chain
  uint16_t* node_in;       // [M, conv_dim] bf16: tree nodes' conv inputs (for the commit)
  int* tinfo;              // [3, 32] workspace: the tree's processing order, depths, branch flags
  long slot_stride;        // floats
  int ld, hidden, M, H, HV, R;
  float eps, scale;
};

__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : logf(1.f + expf(x)); }
// silu(x) = x / (1 + e^-x) with the hardware's 2^x and reciprocal (about 1 ulp each; the
// results are rounded to bf16): three instructions where expf and an IEEE divide take ~25.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gdn_rsrc(const void* p, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p, (short)0, (int)bytes, 0x00020000);
}

// ------------------------------------------------------------------ tree helpers

// Parent of node t of a draft tree (parent[t] < t; node 0 is the root). A parent outside
// 0..t-1 reads as the root, so every walk up the tree ends within t steps.
__device__ __forceinline__ int tree_parent(const int32_t* parent, int t) {
  const int p = parent[t];
  return (p >= 0 && p < t) ? p : 0;
}

// The order the recurrence visits a tree's nodes in: depth first, children by index (each node
// right after its parent or after the subtree of an earlier sibling), computed by threads
// 0..M-1 of one workgroup. Node t's position is depth(t) plus, for every node a != root on its
// root path, the sizes of a's earlier siblings' subtrees. Writes order[32] | depth[32] | branch
// flags[32] (1 for a node with two or more children: its state is visited again) to info.
__device__ void tree_order(const int32_t* parent, int M, int* info) {
  __shared__ int tp[32], tsz[32], tesz[32];
  __shared__ uint32_t tanc[32];
  const int t = threadIdx.x;
  const bool node = t < M;
  if (node) tp[t] = t == 0 ? -1 : tree_parent(parent, t);
  __syncthreads();
  int dep = 0;
  uint32_t anc = node ? 1u << t : 0u;
  if (node)
    for (int j = t; j > 0; ++dep) {
      j = tp[j];
      anc |= 1u << j;
    }
  if (node) tanc[t] = anc;
  __syncthreads();
  int size = 0, kids = 0;
  if (node)
    for (int u = 0; u < M; ++u) {
      size += (tanc[u] >> t) & 1u;
      kids += tp[u] == t;
    }
  if (node) tsz[t] = size;
  __syncthreads();
  int esz = 0;
  if (node && t > 0)
    for (int u = 1; u < t; ++u) esz += tp[u] == tp[t] ? tsz[u] : 0;
  if (node) tesz[t] = esz;
  __syncthreads();
  if (node) {
    int pre = dep;
    for (uint32_t m = anc & ~1u; m; m &= m - 1) pre += tesz[__builtin_ctz(m)];
    info[pre] = t;
    info[32 + t] = dep;
    info[64 + t] = kids >= 2;
  }
}

// ------------------------------------------------------------------ prep: conv, norms, gates

template <int MAXM, bool TREE>
__global__ __launch_bounds__(kGdnThreads) void gdn_prep_kernel(GdnArgs a) {
  constexpr int TG = gdn_tg<MAXM>();
  __shared__ float part[4][8];
  __shared__ float ssq[4][TG];
  __shared__ int src_s[MAXM][3];  // window inputs of token t, 1..3 back: a token, or -(ring slot + 1)
  __shared__ int par_l[MAXM];     // a tree's parents, loaded once (the walks below run in LDS)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int M = a.M;
  const int QK = a.H * kGdnK;
  const int C = 2 * QK + a.HV * kGdnV;
  const int n_cb = (C + kGdnThreads - 1) / kGdnThreads;
  const int n_conv = n_cb * ((M + TG - 1) / TG);
  if (TREE && blockIdx.x == gridDim.x - 1) {
    tree_order(a.parent, M, a.tinfo);
    return;
  }
  if ((int)blockIdx.x < n_conv) {
    // One conv channel per thread for TG tokens; a workgroup's 256 channels are two whole q or
    // k heads (QK is a multiple of 256) or 256 v channels. The window of token t holds the inputs
    // 1..3 back on its path: the previous tokens of a chain, a tree node's ancestors, and the
    // ring's committed positions pos - 1 .. pos - 3 where the path is shorter.
    const int cb = blockIdx.x % n_cb, t0 = TG * (blockIdx.x / n_cb);
    const int ch = cb * kGdnThreads + tid;
    const bool on = ch < C;
    const int pr = (int)(*a.pos % a.R);  // ring column of token 0
    // A tree's windows come from ancestors that the parent walks below name: every node's input
    // of this channel is loaded first (independent of the tree's shape, so the loads' latency
    // runs under the walks) and staged in LDS, where the windows read them.
    __shared__ uint16_t nv_s[TREE ? MAXM : 1][kGdnThreads];
    uint16_t nv[TREE ? MAXM : 1];
    // The parents first (the walks wait for them, and vector loads complete in issue order), then
    // the conv weights and the ring's committed inputs. Every thread loads, at a clamped channel
    // (a load under a branch would be waited for where the paths meet).
    const int chc = on ? ch : C - 1;
    const int par_raw = TREE ? a.parent[min(tid, M - 1)] : 0;
    asm volatile("" ::: "memory");  // issued before the loads below
    const uint2 wu = *(const uint2*)(a.conv_w + (size_t)chc * 4);
    uint16_t* rrow = a.ring + (size_t)chc * a.R;
    uint16_t rr[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) rr[j] = rrow[(pr + j - 3 + a.R) % a.R];  // pos - 3 + j
    if (TREE) {
#pragma unroll
      for (int u = 0; u < MAXM; ++u) nv[u] = a.qkvz[(size_t)min(u, M - 1) * a.ld + chc];
      if (tid < M) par_l[tid] = tid > 0 && par_raw >= 0 && par_raw < tid ? par_raw : 0;  // tree_parent's rule
      lds_barrier();
    }
    if (TREE && tid < M) {
      int j = tid, dep = 0;
      for (int s = 0; s < MAXM && j > 0; ++s) {
        j = par_l[j];
        ++dep;
      }
      j = tid;
      for (int k = 0; k < 3; ++k) {  // k + 1 back
        if (dep > k) {
          j = par_l[j];
          src_s[tid][k] = j;
        } else {
          src_s[tid][k] = -(3 - (k + 1 - dep)) - 1;  // position pos - (k + 1 - dep): ring slot 3 - (k + 1 - dep)
        }
      }
    }
    if (TREE) {
#pragma unroll
      for (int u = 0; u < MAXM; ++u) nv_s[u][tid] = nv[u];
      lds_barrier();
    }
    float y[TG];
#pragma unroll
    for (int u = 0; u < TG; ++u) y[u] = 0.f;
    if (on) {
      const float w0 = bf16_bits_to_f32(wu.x & 0xFFFFu), w1 = bf16_bits_to_f32(wu.x >> 16);
      const float w2 = bf16_bits_to_f32(wu.y & 0xFFFFu), w3 = bf16_bits_to_f32(wu.y >> 16);
      // the tokens' own inputs and (trees) the windows', every load first
      float win[TG + 3];  // chain: positions pos - 3 .. pos + TG - 1
      uint16_t xin[TG], wt[TG][3];
#pragma unroll
      for (int j = 0; j < 3; ++j) win[j] = bf16_bits_to_f32(rr[j]);
#pragma unroll
      for (int u = 0; u < TG; ++u) {
        const int t = min(t0 + u, M - 1);
        xin[u] = TREE ? nv_s[t][tid] : a.qkvz[(size_t)t * a.ld + ch];
        win[u + 3] = bf16_bits_to_f32(t0 + u < M ? xin[u] : (uint16_t)0);
        if (TREE)
#pragma unroll
          for (int k = 0; k < 3; ++k) {
            const int sn = src_s[t][k];
            wt[u][k] = sn >= 0 ? nv_s[sn][tid] : (uint16_t)0;
          }
      }
#pragma unroll
      for (int u = 0; u < TG; ++u) {
        const int t = t0 + u;
        if (t < M) {
          // oldest first: 3 back, 2 back, 1 back, the token itself (a chain's group starts at
          // token 0, so its window is win[u .. u + 3])
          float sv[3] = {win[u + 2], win[u + 1], win[u]};
          if (TREE)
#pragma unroll
            for (int k = 0; k < 3; ++k) {
              const int sn = src_s[t][k];
              sv[k] = sn >= 0 ? bf16_bits_to_f32(wt[u][k]) : win[-sn - 1];
            }
          float yv = sv[2] * w0;
          yv = yv + sv[1] * w1;
          yv = yv + sv[0] * w2;
          yv = yv + bf16_bits_to_f32(xin[u]) * w3;
          yv = bf16r(yv);
          y[u] = bf16r(silu_fast(yv));
        }
      }
      if (TREE) {  // a tree's inputs wait for the commit
#pragma unroll
        for (int u = 0; u < TG; ++u)
          if (t0 + u < M) a.node_in[(size_t)(t0 + u) * C + ch] = xin[u];
      } else {  // a chain's go to the ring, after every read of it
#pragma unroll
        for (int u = 0; u < TG; ++u)
          if (t0 + u < M) rrow[(pr + t0 + u) % a.R] = xin[u];
      }
    }
    if (cb * kGdnThreads >= 2 * QK) {  // v channels: stored as they are
      if (on)
#pragma unroll
        for (int u = 0; u < TG; ++u)
          if (t0 + u < M) a.vconv[(size_t)(t0 + u) * a.HV * kGdnV + (ch - 2 * QK)] = f32_to_bf16_bits(y[u]);
      return;
    }
    // q or k: normalise each token's 128-channel head (waves 0-1: first head, 2-3: second)
#pragma unroll
    for (int u = 0; u < TG; ++u) {
      const float sq = sum_wave(y[u] * y[u]);
      if (lane == 0) ssq[wave][u] = sq;
    }
    __syncthreads();
    const bool isq = ch < QK;
    const int hb = wave & ~1;  // first wave of this head
#pragma unroll
    for (int u = 0; u < TG; ++u) {
      if (t0 + u < M) {
        const float n = sqrtf((ssq[hb][u] + ssq[hb + 1][u]) + 1e-6f);
        a.qk[(size_t)(t0 + u) * 2 * QK + ch] = isq ? y[u] / n * a.scale : y[u] / n;
      }
    }
    return;
  }
  // gate row r of ba_w (b for r < HV, a for r >= HV) for one group of 8 tokens
  const int r = (blockIdx.x - n_conv) % (2 * a.HV), t0 = 8 * ((blockIdx.x - n_conv) / (2 * a.HV));
  const int q0 = a.hidden / 4 * wave, q1 = a.hidden / 4 * (wave + 1);
  const auto xr = gdn_rsrc(a.x, (size_t)M * a.hidden * 2);
  const uint16_t* wrow = a.ba_w + (size_t)r * a.hidden;
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  constexpr int kCh = 3;
  const auto wr = gdn_rsrc(wrow, (size_t)a.hidden * 2);
  {
    float acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = 0.f;
    // three 512-element chunks per pass (a quarter of hidden 5120 is 2.5), every load of a pass
    // issued first; chunks past the quarter load zeros (offsets beyond the buffer resources)
    for (int e = q0 + 8 * lane; e < q1; e += kCh * 8 * 64) {
      u4 wv[kCh], xv[kCh][8];
#pragma unroll
      for (int c = 0; c < kCh; ++c) {
        const int ec = e + c * 8 * 64;
        const bool in = ec < q1;
        wv[c] = __builtin_amdgcn_raw_buffer_load_b128(wr, in ? ec * 2 : 0x7FFFFFF0, 0, 0);
#pragma unroll
        for (int t = 0; t < 8; ++t)
          xv[c][t] = __builtin_amdgcn_raw_buffer_load_b128(xr, (in && t0 + t < M) ? ((t0 + t) * a.hidden + ec) * 2
                                                                                   : 0x7FFFFFF0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < kCh; ++c) {
        const uint32_t wa[4] = {wv[c].x, wv[c].y, wv[c].z, wv[c].w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const uint32_t xw[4] = {xv[c][t].x, xv[c][t].y, xv[c][t].z, xv[c][t].w};
#pragma unroll
          for (int q = 0; q < 4; ++q)
            acc[t] += bf16_bits_to_f32(xw[q] & 0xFFFFu) * bf16_bits_to_f32(wa[q] & 0xFFFFu) +
                      bf16_bits_to_f32(xw[q] >> 16) * bf16_bits_to_f32(wa[q] >> 16);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float v = sum_wave(acc[t]);
      if (lane == 0) part[wave][t] = v;
    }
    __syncthreads();
    if (tid < 8 && t0 + tid < M)
      a.gates[(size_t)(t0 + tid) * 2 * a.HV + r] = bf16r(((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid]);
  }
}

// ------------------------------------------------------------------ step: the recurrence

template <int MAXM, bool TREE>
__global__ __launch_bounds__(kGdnThreads) void gdn_step_kernel(GdnArgs a) {
  __shared__ float cq[MAXM][kGdnK], ck[MAXM][kGdnK], cv[MAXM][kGdnBV];
  __shared__ float beta_s[MAXM], decay_s[MAXM];
  __shared__ int par_s[MAXM], ord_s[MAXM], dep_s[MAXM], br_s[MAXM];
  __shared__ float2 red[2][4][8];
  __shared__ __attribute__((aligned(16))) float4 red4[2][4][8];  // [buffer][wave][column pair]: o.x, o.y, kv.x, kv.y
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hv = blockIdx.x / kGdnNVB, vb = blockIdx.x % kGdnNVB;
  const int ih = hv / (a.HV / a.H);
  const int M = a.M;
  const int QK = a.H * kGdnK, VAL = a.HV * kGdnV;
  const int64_t slot = *a.slot;
  const int vq = lane & 7, kg = lane >> 3;
  const int c0 = 2 * vq;                    // this lane's first column within the block
  const int v0 = vb * kGdnBV + c0;          // ... within the head
  const int k0 = 32 * wave + 4 * kg;        // this lane's first row

  // prologue: the committed state tile, then this block's normalised q / k, v and gates
  float2 S[4];
  {
    const float* src = a.rec + slot * a.slot_stride + (size_t)hv * kGdnK * kGdnV + v0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // non-temporal: read once
      const float* r = src + (size_t)(k0 + j) * kGdnV;
      S[j] = make_float2(__builtin_nontemporal_load(r), __builtin_nontemporal_load(r + 1));
    }
  }
  // q / k, v and the gates: every load issued at once (a loop with a runtime bound waited for
  // each iteration's loads); indices past M are clamped to token M - 1 and not stored
  {
    constexpr int kQK = MAXM * kGdnK / kGdnThreads;
    float qv[kQK], kv2[kQK];
#pragma unroll
    for (int q = 0; q < kQK; ++q) {
      const int e = tid + kGdnThreads * q, t = min(e / kGdnK, M - 1), c = e % kGdnK;
      qv[q] = a.qk[(size_t)t * 2 * QK + ih * kGdnK + c];
      kv2[q] = a.qk[(size_t)t * 2 * QK + QK + ih * kGdnK + c];
    }
    constexpr int kVE = (MAXM * kGdnBV + kGdnThreads - 1) / kGdnThreads;  // v elements per thread
    uint16_t vraw[kVE];
#pragma unroll
    for (int q = 0; q < kVE; ++q) {
      const int ev = min(tid + kGdnThreads * q, MAXM * kGdnBV - 1), tv = min(ev / kGdnBV, M - 1);
      vraw[q] = a.vconv[(size_t)tv * VAL + hv * kGdnV + vb * kGdnBV + ev % kGdnBV];
    }
    const int tg = min(tid, M - 1);
    const float b = a.gates[(size_t)tg * 2 * a.HV + hv];
    const float av = a.gates[(size_t)tg * 2 * a.HV + a.HV + hv];
#pragma unroll
    for (int q = 0; q < kQK; ++q) {
      const int e = tid + kGdnThreads * q, t = e / kGdnK, c = e % kGdnK;
      if (t < M) {
        cq[t][c] = qv[q];
        ck[t][c] = kv2[q];
      }
    }
#pragma unroll
    for (int q = 0; q < kVE; ++q) {
      const int ev = tid + kGdnThreads * q;
      if (ev < MAXM * kGdnBV && ev / kGdnBV < M) cv[ev / kGdnBV][ev % kGdnBV] = bf16_bits_to_f32(vraw[q]);
    }
    if (tid < M) {
      beta_s[tid] = bf16r(1.f / (1.f + expf(-b)));
      decay_s[tid] = expf(a.A[hv] * softplus_f(av + a.dt_bias[hv]));
      par_s[tid] = TREE && tid > 0 ? tree_parent(a.parent, tid) : tid - 1;
      ord_s[tid] = TREE ? a.tinfo[tid] : tid;
      dep_s[tid] = TREE ? a.tinfo[32 + tid] : tid;
      br_s[tid] = TREE ? a.tinfo[64 + tid] : 0;
    }
  }
  __syncthreads();

  // the recurrence. With kv_t = sum_k S_{t-1}[k] k_t[k] (S before token t's decay):
  //   dv = beta_t (v_t - e^{g_t} kv_t),  S_t = S_{t-1} e^{g_t} + k_t dv^T,  o_t = q_t^T S_t,
  // and kv_{t+1} is summed together with o_t, so each token costs one cross-wave exchange.
  // Sums over k: a lane's 4 rows, the wave's 8 row groups (lane ^ 8, ^ 16, ^ 32), the 4 waves.
  auto ksum = [](float v) { return sum_x32(sum_x16(sum_x8(v))); };
  auto wsum = [&](float2 p, int buf) {  // every lane of every wave must call it
    p = make_float2(ksum(p.x), ksum(p.y));
    if (kg == 0) red[buf][wave][vq] = p;
    __syncthreads();
    float2 r = red[buf][0][vq];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float2 u = red[buf][w][vq];
      r.x += u.x;
      r.y += u.y;
    }
    return r;
  };
  // Nodes in the visiting order (a chain: 0..M-1; a tree: depth first). The state a node starts
  // from is the previous node's, or -- for a tree node whose parent is not the previous node --
  // the parent's, kept in a register stack by depth when the parent has several children (a
  // load of the parent's snapshot would wait for every store still in flight). Parents deeper
  // than the stack reload their snapshot.
  constexpr int kStk = TREE ? 8 : 1;
  float2 stk[kStk][4];
  float2 kv;
  {
    float2 p = make_float2(0.f, 0.f);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float kk = ck[0][k0 + j];
      p.x = fmaf(S[j].x, kk, p.x);
      p.y = fmaf(S[j].y, kk, p.y);
    }
    kv = wsum(p, 0);
  }
  float* const obase = a.o_ws + (size_t)hv * kGdnV + v0;
  const size_t head_off = (size_t)hv * kGdnK * kGdnV + v0;
  if constexpr (TREE) {
    // Each node's wave-uniform values (its index in the visiting order, the next node, the node
    // that one continues from, depths, branch flag, beta and the decay) sit in lane i of a
    // register for visit i (M <= 32 lanes), read with v_readlane: the loop makes no LDS round
    // trip for them, where a readfirstlane of an LDS value stalled the wave (one per SIMD) for
    // each. The node's rows of v, k and q and the next node's k row are read from LDS one visit
    // ahead, under the previous visit's work.
    int T_l = 0, TN_l = 0, PN_l = 0, DT_l = 0, BT_l = 0, DPN_l = 0;
    float BE_l = 0.f, EG_l = 0.f;
    if (lane < M) {
      T_l = TREE ? ord_s[lane] : lane;
      TN_l = lane + 1 < M ? (TREE ? ord_s[lane + 1] : lane + 1) : T_l;
      PN_l = TREE && lane + 1 < M ? par_s[TN_l] : T_l;
      if (TREE) {
        DT_l = dep_s[T_l];
        BT_l = br_s[T_l];
        DPN_l = dep_s[PN_l];
      }
      BE_l = beta_s[T_l];
      EG_l = decay_s[T_l];
    }
    auto lane_i = [](int v, int i) { return __builtin_amdgcn_readlane(v, i); };
    auto lane_f = [](float v, int i) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i)); };
    // visit 0's rows
    float2 vt;
    float kk[4], qq[4], kn[4];
    {
      const int t = lane_i(T_l, 0), tn = lane_i(TN_l, 0);
      vt = *(const float2*)&cv[t][c0];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kk[j] = ck[t][k0 + j];
        qq[j] = cq[t][k0 + j];
        kn[j] = ck[tn][k0 + j];
      }
    }
    for (int i = 0; i < M; ++i) {
      const int t = lane_i(T_l, i), tn = lane_i(TN_l, i);
      const int pn = TREE ? lane_i(PN_l, i) : t;  // the node the next one continues from
      const float beta = lane_f(BE_l, i), eg = lane_f(EG_l, i);
      float2 dv;
      dv.x = beta * fmaf(-eg, kv.x, vt.x);
      dv.y = beta * fmaf(-eg, kv.y, vt.y);
      // the next visit's rows (its node is tn; its next node's k row), read under this visit's work
      float2 vt1;
      float qq1[4], kn1[4];
      {
        const int tn1 = lane_i(TN_l, i + 1 < M ? i + 1 : i);
        vt1 = *(const float2*)&cv[tn][c0];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          qq1[j] = cq[tn][k0 + j];
          kn1[j] = ck[tn1][k0 + j];
        }
      }
      float2 o = make_float2(0.f, 0.f), nx = o;
      float* dst = a.rec + (size_t)t * a.slot_stride + head_off;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        S[j].x = fmaf(kk[j], dv.x, __fmul_rn(S[j].x, eg));
        S[j].y = fmaf(kk[j], dv.y, __fmul_rn(S[j].y, eg));
        // non-temporal: of the M snapshots only the accepted one is read again (by the next step)
        __builtin_nontemporal_store(S[j].x, dst + (size_t)(k0 + j) * kGdnV);
        __builtin_nontemporal_store(S[j].y, dst + (size_t)(k0 + j) * kGdnV + 1);
        o.x = fmaf(S[j].x, qq[j], o.x);
        o.y = fmaf(S[j].y, qq[j], o.y);
      }
      if (TREE && lane_i(BT_l, i)) {  // a branch node, visited again for its later children
        const int d = lane_i(DT_l, i);
#pragma unroll
        for (int e = 0; e < kStk; ++e)
          if (e == d)
#pragma unroll
            for (int j = 0; j < 4; ++j) stk[e][j] = S[j];
      }
      // the next node's k product from the state it starts from: this node's, or an earlier one's.
      // The snapshot-load path waits for its loads itself: a load still pending where the paths
      // meet would make every path wait for the memory counter, i.e. for this node's stores.
      auto next_sum = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          nx.x = fmaf(S[j].x, kn[j], nx.x);
          nx.y = fmaf(S[j].y, kn[j], nx.y);
        }
      };
      if (!TREE || pn == t) {
        next_sum();
      } else {
        const int d = lane_i(DPN_l, i);
        if (d < kStk) {
#pragma unroll
          for (int e = 0; e < kStk; ++e)
            if (e == d)
#pragma unroll
              for (int j = 0; j < 4; ++j) S[j] = stk[e][j];
          next_sum();
        } else {
          const float* src = a.rec + (size_t)pn * a.slot_stride + head_off;
#pragma unroll
          for (int j = 0; j < 4; ++j) S[j] = *(const float2*)(src + (size_t)(k0 + j) * kGdnV);
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) here, so the paths meet with no load pending
          next_sum();
        }
      }
      // both sums in one exchange: buffer (i + 1) % 2 alternates so the next node's writes never
      // race this node's reads (the barrier between them separates them)
      // the four sums in one pass: lane row j (lanes 16 j ..) holds o.x, o.y, nx.x, nx.y for j = 0..3
      const float tot = sum_x8_16_32_4(o.x, o.y, nx.x, nx.y);
      const int buf = (i + 1) & 1;
      if ((kg & 1) == 0) ((float*)&red4[buf][wave][vq])[kg >> 1] = tot;
      __syncthreads();
      float4 r4 = red4[buf][0][vq];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float4 u = red4[buf][w][vq];
        r4.x += u.x;
        r4.y += u.y;
        r4.z += u.z;
        r4.w += u.w;
      }
      const float2 ro = make_float2(r4.x, r4.y), rn = make_float2(r4.z, r4.w);
      kv = rn;
      if (wave == 0 && kg == 0) {
        float* op = obase + (size_t)t * VAL;
        ws_st(op + 0, bf16r(ro.x));
        ws_st(op + 1, bf16r(ro.y));
      }
      // the next visit's rows: its k row is this visit's next-node row
      vt = vt1;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        kk[j] = kn[j];
        qq[j] = qq1[j];
        kn[j] = kn1[j];
      }
    }
  } else {  // a chain: node i is token i, and its values are read where they are used
    for (int i = 0; i < M; ++i) {
      // wave-uniform values from LDS, kept in scalar registers
      const int t = TREE ? __builtin_amdgcn_readfirstlane(ord_s[i]) : i;
      const int tn = i + 1 < M ? (TREE ? __builtin_amdgcn_readfirstlane(ord_s[i + 1]) : i + 1) : t;  // the next node
      const int pn = TREE && i + 1 < M ? __builtin_amdgcn_readfirstlane(par_s[tn]) : t;  // ... continues from
      const float beta = beta_s[t], eg = decay_s[t];
      const float* vt = &cv[t][c0];
      float2 dv;
      dv.x = beta * fmaf(-eg, kv.x, vt[0]);
      dv.y = beta * fmaf(-eg, kv.y, vt[1]);
      float2 o = make_float2(0.f, 0.f), nx = o;
      float* dst = a.rec + (size_t)t * a.slot_stride + head_off;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float kk = ck[t][k0 + j], qq = cq[t][k0 + j];
        S[j].x = fmaf(kk, dv.x, __fmul_rn(S[j].x, eg));
        S[j].y = fmaf(kk, dv.y, __fmul_rn(S[j].y, eg));
        // non-temporal: of the M snapshots only the accepted one is read again (by the next step)
        __builtin_nontemporal_store(S[j].x, dst + (size_t)(k0 + j) * kGdnV);
        __builtin_nontemporal_store(S[j].y, dst + (size_t)(k0 + j) * kGdnV + 1);
        o.x = fmaf(S[j].x, qq, o.x);
        o.y = fmaf(S[j].y, qq, o.y);
      }
      if (TREE && __builtin_amdgcn_readfirstlane(br_s[t])) {  // a branch node, visited again for its later children
        const int d = __builtin_amdgcn_readfirstlane(dep_s[t]);
#pragma unroll
        for (int e = 0; e < kStk; ++e)
          if (e == d)
#pragma unroll
            for (int j = 0; j < 4; ++j) stk[e][j] = S[j];
      }
      // the next node's k product from the state it starts from: this node's, or an earlier one's.
      // The snapshot-load path waits for its loads itself: a load still pending where the paths
      // meet would make every path wait for the memory counter, i.e. for this node's stores.
      auto next_sum = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float kn = ck[tn][k0 + j];
          nx.x = fmaf(S[j].x, kn, nx.x);
          nx.y = fmaf(S[j].y, kn, nx.y);
        }
      };
      if (!TREE || pn == t) {
        next_sum();
      } else {
        const int d = __builtin_amdgcn_readfirstlane(dep_s[pn]);
        if (d < kStk) {
#pragma unroll
          for (int e = 0; e < kStk; ++e)
            if (e == d)
#pragma unroll
              for (int j = 0; j < 4; ++j) S[j] = stk[e][j];
          next_sum();
        } else {
          const float* src = a.rec + (size_t)pn * a.slot_stride + head_off;
#pragma unroll
          for (int j = 0; j < 4; ++j) S[j] = *(const float2*)(src + (size_t)(k0 + j) * kGdnV);
          __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0) here, so the paths meet with no load pending
          next_sum();
        }
      }
      // both sums in one exchange: buffer (i + 1) % 2 alternates so the next node's writes never
      // race this node's reads (the barrier inside wsum separates them)
      // the four sums in one pass: lane row j (lanes 16 j ..) holds o.x, o.y, nx.x, nx.y for j = 0..3
      const float tot = sum_x8_16_32_4(o.x, o.y, nx.x, nx.y);
      const int buf = (i + 1) & 1;
      if ((kg & 1) == 0) ((float*)&red4[buf][wave][vq])[kg >> 1] = tot;
      __syncthreads();
      float4 r4 = red4[buf][0][vq];
#pragma unroll
      for (int w = 1; w < 4; ++w) {
        const float4 u = red4[buf][w][vq];
        r4.x += u.x;
        r4.y += u.y;
        r4.z += u.z;
        r4.w += u.w;
      }
      const float2 ro = make_float2(r4.x, r4.y), rn = make_float2(r4.z, r4.w);
      kv = rn;
      if (wave == 0 && kg == 0) {
        float* op = obase + (size_t)t * VAL;
        ws_st(op + 0, bf16r(ro.x));
        ws_st(op + 1, bf16r(ro.y));
      }
    }
  }

  // The last of the head's column blocks applies the gated norm to all V columns, every token.
  // Its z and gain loads are issued before the arrival count.
  const int Z = 2 * QK + VAL;
  constexpr int kZU = MAXM / 4;  // tokens per wave in the norm
  uint32_t zb[kZU][2];
#pragma unroll
  for (int u = 0; u < kZU; ++u) {
    const int t = wave + 4 * u;
    const uint16_t* zr = a.qkvz + (size_t)t * a.ld + Z + (size_t)hv * kGdnV;
    zb[u][0] = t < M ? zr[lane] : 0u;
    zb[u][1] = t < M ? zr[lane + 64] : 0u;
  }
  const float nw0 = bf16_bits_to_f32(a.norm_w[lane]), nw1 = bf16_bits_to_f32(a.norm_w[lane + 64]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    int* c = a.cnt + hv * 32;
    handoff_release();
    const int old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == kGdnNVB - 1;
    if (last) {
      __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      handoff_acquire();
    }
  }
  __syncthreads();
  if (!last) return;
#pragma unroll
  for (int u = 0; u < kZU; ++u) {
    const int t = wave + 4 * u;
    if (t >= M) break;
    const float* op = a.o_ws + (size_t)t * VAL + (size_t)hv * kGdnV;
    const float o0 = ws_ld(op + lane), o1 = ws_ld(op + lane + 64);
    const float var = sum_wave(o0 * o0 + o1 * o1) / (float)kGdnV;
    const float r = 1.f / sqrtf(var + a.eps);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float ob = h ? o1 : o0;
      const float n = bf16r(bf16r(ob * r) * (h ? nw1 : nw0));
      const float z = bf16_bits_to_f32(zb[u][h]);
      a.y[(size_t)t * VAL + (size_t)hv * kGdnV + lane + 64 * h] = f32_to_bf16_bits(n * silu_fast(z));
    }
  }
}

}  // namespace tr

using namespace tr;

extern "C" {

// Workspace: kGdnMaxHV arrival counters (one per 128-byte line) in a fixed region at offset 0,
// then the head outputs [M, HV V] fp32, normalised q | k [M, 2 H K] fp32, the v conv outputs
// [M, HV V] bf16, the gates [M, 2 HV] fp32 and a tree's visiting order, each 256-byte aligned. The counters' place does
// not depend on the call's shape, so one zero-filled buffer serves calls of every shape (a
// shape-dependent layout let one shape's head outputs land on another shape's counters).
constexpr int kGdnMaxHV = 256;
static size_t gdn_ws_part(size_t bytes) { return (bytes + 255) / 256 * 256; }

size_t tr_gdn_workspace_bytes(int M, int H, int HV) {
  if (M < 1 || M > kGdnMaxTree || H < 1 || HV < 1 || HV > kGdnMaxHV) return 0;
  return gdn_ws_part((size_t)kGdnMaxHV * 32 * sizeof(int)) + gdn_ws_part((size_t)M * HV * kGdnV * sizeof(float)) +
         gdn_ws_part((size_t)M * 2 * H * kGdnK * sizeof(float)) + gdn_ws_part((size_t)M * HV * kGdnV * 2) +
         gdn_ws_part((size_t)M * 2 * HV * sizeof(float)) + gdn_ws_part(3 * 32 * sizeof(int));
}

}  // extern "C"

namespace {

// Shared by the chain and tree entry points: the shape checks past M, the workspace carve-up and
// the two launches (8-token kernels up to M = 8, 32-token kernels above).
int gdn_launch(const void* qkvz, int ld, const void* x, const void* ba_w, void* ring, const void* conv_w,
               const float* A, const float* dt_bias, float* rec, long slot_stride, const int64_t* slot,
               const void* norm_w, const int64_t* pos, void* y, void* workspace, size_t workspace_bytes, int M,
               int H, int HV, int K, int V, int hidden, int R, float eps, const int32_t* parent, void* node_in,
               void* stream) {
  if (K != kGdnK || V != kGdnV || H < 1 || HV < H || HV > kGdnMaxHV || HV % H || (2 * H * K) % kGdnThreads ||
      hidden < 32 || hidden % 32 || R < 3)
    return TR_ERR_SHAPE;
  if (!qkvz || !x || !ba_w || !ring || !conv_w || !A || !dt_bias || !rec || !slot || !norm_w || !pos || !y ||
      !workspace)
    return TR_ERR_ARG;
  if (ld < 2 * H * K + 2 * HV * V || slot_stride < (long)HV * K * V) return TR_ERR_ARG;
  if (workspace_bytes < tr_gdn_workspace_bytes(M, H, HV)) return TR_ERR_ARG;
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
  char* w = (char*)workspace;
  a.cnt = (int*)w;
  w += gdn_ws_part((size_t)kGdnMaxHV * 32 * sizeof(int));
  a.o_ws = (float*)w;
  w += gdn_ws_part((size_t)M * HV * kGdnV * sizeof(float));
  a.qk = (float*)w;
  w += gdn_ws_part((size_t)M * 2 * H * K * sizeof(float));
  a.vconv = (uint16_t*)w;
  w += gdn_ws_part((size_t)M * HV * V * 2);
  a.gates = (float*)w;
  w += gdn_ws_part((size_t)M * 2 * HV * sizeof(float));
  a.tinfo = (int*)w;
  a.parent = parent;
  a.node_in = (uint16_t*)node_in;
  a.slot_stride = slot_stride;
  a.ld = ld;
  a.hidden = hidden;
  a.M = M;
  a.H = H;
  a.HV = HV;
  a.R = R;
  a.eps = eps;
  a.scale = 1.f / sqrtf((float)K);
  const int C = 2 * H * K + HV * V;
  // prep: one workgroup per (256 conv channels, group of TG tokens), one per (gate row, group
  // of 8 tokens), and for a tree one that works out the visiting order
  const int TG = M <= kGdnMaxM ? gdn_tg<kGdnMaxM>() : gdn_tg<kGdnMaxTree>();
  const dim3 prep_grid((C + kGdnThreads - 1) / kGdnThreads * ((M + TG - 1) / TG) + 2 * HV * ((M + 7) / 8) +
                       (parent ? 1 : 0));
  const dim3 step_grid(HV * kGdnNVB), block(kGdnThreads);
  hipStream_t st = (hipStream_t)stream;
  if (M <= kGdnMaxM && !parent) {
    hipLaunchKernelGGL((gdn_prep_kernel<kGdnMaxM, false>), prep_grid, block, 0, st, a);
    if (hipGetLastError() != hipSuccess) return TR_ERR_LAUNCH;
    hipLaunchKernelGGL((gdn_step_kernel<kGdnMaxM, false>), step_grid, block, 0, st, a);
  } else if (M <= kGdnMaxM) {
    hipLaunchKernelGGL((gdn_prep_kernel<kGdnMaxM, true>), prep_grid, block, 0, st, a);
    if (hipGetLastError() != hipSuccess) return TR_ERR_LAUNCH;
    hipLaunchKernelGGL((gdn_step_kernel<kGdnMaxM, true>), step_grid, block, 0, st, a);
  } else {
    hipLaunchKernelGGL((gdn_prep_kernel<kGdnMaxTree, true>), prep_grid, block, 0, st, a);
    if (hipGetLastError() != hipSuccess) return TR_ERR_LAUNCH;
    hipLaunchKernelGGL((gdn_step_kernel<kGdnMaxTree, true>), step_grid, block, 0, st, a);
  }
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

// Tree commit of the conv rings: ring column (base + d) % R <- node_in[commit[d]] for the
// accepted path d = 0..n in order (base = pos - n - 1, pos already advanced by the accept), so
// the ring ends as a chain step over the path would leave it. One thread per (layer, channel).
// A path that names a node outside 0..M-1 or is longer than M commits nothing and sets *status.
__global__ void gdn_tree_commit_kernel(uint16_t* ring, long ring_stride, const uint16_t* node_in, long node_stride,
                                       int layers, int C, int R, int M, const int64_t* pos,
                                       const int64_t* n_accepted, const int64_t* commit, int* status) {
  const int ch = blockIdx.x * blockDim.x + threadIdx.x, layer = blockIdx.y;
  const int n = (int)*n_accepted;
  const int64_t base = *pos - n - 1;
  bool bad = n < 0 || n >= M || base < 0;
  for (int d = 0; d <= n && d < M; ++d) bad |= commit[d] < 0 || commit[d] >= M;
  if (bad) {
    if (status && ch == 0 && layer == 0) *status = 1;
    return;
  }
  if (ch >= C || layer >= layers) return;
  uint16_t* rrow = ring + (size_t)layer * ring_stride + (size_t)ch * R;
  const uint16_t* src = node_in + (size_t)layer * node_stride + ch;
  for (int d = 0; d <= n; ++d) rrow[(base + d) % R] = src[(size_t)commit[d] * C];
}

}  // namespace

extern "C" {

int tr_gdn_step(const void* qkvz, int ld, const void* x, const void* ba_w, void* ring, const void* conv_w,
                const float* A, const float* dt_bias, float* rec, long slot_stride, const int64_t* slot,
                const void* norm_w, const int64_t* pos, void* y, void* workspace, size_t workspace_bytes, int M,
                int H, int HV, int K, int V, int hidden, int R, float eps, void* stream) {
  if (M == 0) return TR_OK;
  if (M < 0 || M > kGdnMaxM || R < M + 3) return TR_ERR_SHAPE;
  return gdn_launch(qkvz, ld, x, ba_w, ring, conv_w, A, dt_bias, rec, slot_stride, slot, norm_w, pos, y, workspace,
                    workspace_bytes, M, H, HV, K, V, hidden, R, eps, nullptr, nullptr, stream);
}

int tr_gdn_tree_step(const void* qkvz, int ld, const void* x, const void* ba_w, const void* ring, const void* conv_w,
                     const float* A, const float* dt_bias, float* rec, long slot_stride, const int64_t* slot,
                     const void* norm_w, const int64_t* pos, const int32_t* parent, void* node_in, void* y,
                     void* workspace, size_t workspace_bytes, int M, int H, int HV, int K, int V, int hidden, int R,
                     float eps, void* stream) {
  if (M == 0) return TR_OK;
  if (M < 0 || M > kGdnMaxTree) return TR_ERR_SHAPE;
  if (!parent || !node_in) return TR_ERR_ARG;
  return gdn_launch(qkvz, ld, x, ba_w, const_cast<void*>(ring), conv_w, A, dt_bias, rec, slot_stride, slot, norm_w,
                    pos, y, workspace, workspace_bytes, M, H, HV, K, V, hidden, R, eps, parent, node_in, stream);
}

int tr_gdn_tree_commit(void* ring, long ring_stride, const void* node_in, long node_stride, int layers, int C, int R,
                       int M, const int64_t* pos, const int64_t* n_accepted, const int64_t* commit, int32_t* status,
                       void* stream) {
  if (layers == 0 || M == 0) return TR_OK;
  if (layers < 0 || C < 1 || R < 1 || M < 1 || M > kGdnMaxTree || ring_stride < (long)C * R ||
      node_stride < (long)M * C)
    return TR_ERR_SHAPE;
  if (!ring || !node_in || !pos || !n_accepted || !commit) return TR_ERR_ARG;
  hipLaunchKernelGGL(gdn_tree_commit_kernel, dim3((C + 255) / 256, layers), dim3(256), 0, (hipStream_t)stream,
                     (uint16_t*)ring, ring_stride, (const uint16_t*)node_in, node_stride, layers, C, R, M, pos,
                     n_accepted, commit, (int*)status);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"
