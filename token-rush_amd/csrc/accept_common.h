// Device helpers shared by the accept kernels (accept.hip) and the GEMM's fused argmax epilogue
// (int4_gemm.hip): agent-scope workspace access, the last-arriver counter, ordered (value, index)
// keys and the verify-step finishes (tokenrush/model.py:302-312, bench/tree_accept.py:91-100).
#pragma once
#include "tr_common.h"

namespace tr {

template <typename T>
__device__ __forceinline__ void ws_st(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T ws_ld(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// True (in every thread) for the workgroup that completes `total` arrivals at *cnt; that
// workgroup also resets the counter. Agent-scope stores made before the call are visible to
// the last arriver's agent-scope loads.
__device__ __forceinline__ bool arrive_last(int* cnt, int total) {
  __shared__ int flag;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    handoff_release();
    const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flag = old == total - 1;
    if (flag) {
      __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      handoff_acquire();
    }
  }
  __syncthreads();
  return flag;
}

// bf16 bits -> unsigned key increasing with the value.
__device__ __forceinline__ uint32_t ord16(uint32_t b) { return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u); }
__device__ __forceinline__ uint32_t unord16(uint32_t k) { return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu); }
// (value, index) -> one 64-bit key: larger value first, then smaller index.
__device__ __forceinline__ uint64_t vkey(uint32_t k16, uint32_t idx) {
  return ((uint64_t)k16 << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ uint32_t vkey_idx(uint64_t k) { return 0xFFFFFFFFu - (uint32_t)k; }

// v of lane l ^ S (S = 1, 2, ..., 32) on the VALU, without the LDS crossbar of __shfl_xor:
// quad_perm for 1 and 2, quad_perm [3,2,1,0] then row_half_mirror for 4 (l -> (l ^ 3) ^ 7),
// row_ror:8 for 8, the permlane swaps for 16 and 32. A swap returns the lane's own value in one
// result and its partner's in the other; taking the one that differs from the own value (or
// either, when they are equal) gives the partner's value. All lanes of the wave must execute it.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int S>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  if constexpr (S == 1) return dpp_u32<0xB1>(v);
  else if constexpr (S == 2) return dpp_u32<0x4E>(v);
  else if constexpr (S == 4) return dpp_u32<0x141>(dpp_u32<0x1B>(v));
  else if constexpr (S == 8) return dpp_u32<0x128>(v);
  else if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return r[0] != v ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return r[0] != v ? r[0] : r[1];
  }
}
template <int S>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
  return ((uint64_t)xor_lane<S>((uint32_t)(v >> 32)) << 32) | xor_lane<S>((uint32_t)v);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  uint64_t w;
  w = xor_lane64<32>(v); v = w > v ? w : v;
  w = xor_lane64<16>(v); v = w > v ? w : v;
  w = xor_lane64<8>(v); v = w > v ? w : v;
  w = xor_lane64<4>(v); v = w > v ? w : v;
  w = xor_lane64<2>(v); v = w > v ? w : v;
  w = xor_lane64<1>(v); v = w > v ? w : v;
  return v;
}

struct AcceptOut {
  int64_t* pred;        // [M] target token per row (may be null)
  int64_t* n_accepted;  // [1]
  int64_t* tok;         // [1] token after the accepted drafts (correction or bonus)
  int64_t* pos;         // [1] device position, advanced by n + 1
  int64_t* slot;        // [1] recurrent-state slot to keep (n for chains, best node for trees)
  int64_t* tokens;      // [M] accepted drafts then tok; -1 beyond
  int64_t* commit;      // [M] chains: positions pos..pos+n; trees: node indices root..best; -1 beyond
};

// Engine._verify_step (tokenrush/model.py:302-312): match = pred[:K] == spec[1:M],
// n = leading matches, tok = pred[n], pos += n + 1, slot = n.
static __device__ __forceinline__ void finish_chain(const int64_t* pred, const int64_t* spec, int M, const AcceptOut& o) {
  // Called by all 64 lanes of one wave: lane i checks draft i + 1 against row i's prediction,
  // n = the first mismatch (a ballot), and lane i writes output i.
  const int i = threadIdx.x & 63;
  const bool miss = i >= M - 1 || pred[i] != spec[i + 1];
  const int n = __builtin_ctzll(__ballot(miss));  // lane M - 1 always misses
  const int64_t t = pred[n];
  const int64_t base = *o.pos;
  if (i < M) {
    o.tokens[i] = i < n ? spec[i + 1] : (i == n ? t : -1);
    o.commit[i] = i <= n ? base + i : -1;
  }
  if (i == 0) {
    *o.n_accepted = n;
    *o.tok = t;
    *o.pos = base + n + 1;
    *o.slot = n;
  }
}

// Longest accepted root path of a draft tree (bench/tree_accept.py:91-100): node 0 is the
// root; node i > 0 (parent[i] < i) is accepted when its token equals the prediction of its
// parent's row and the parent is accepted. Deepest accepted node wins, lowest index on ties. A
// node with a malformed parent (not in 0..i-1) is not accepted, has depth 0, and nothing below
// it is accepted.
//
// Called by all 64 lanes of one wave, lane i = node i (M <= 32). Depth and acceptance come from
// pointer jumping: each lane holds (up, dep, ok) = an ancestor, the edge count to it and the AND
// of the edge checks on the way, and five rounds of "combine with up's triple" reach the root
// (or the malformed node) from depth <= 31. A one-thread walk over the nodes in index order took
// several microseconds of dependent LDS accesses at M = 32.
static __device__ void finish_tree(const int64_t* pred, const int64_t* node_tok, const int32_t* parent, int M,
                                   const AcceptOut& o) {
  const int i = threadIdx.x & 63;
  const bool node = i < M;
  const int p = node && i > 0 ? parent[i] : -1;
  const bool valid = node && i > 0 && p >= 0 && p < i;
  int up = valid ? p : -1;
  int dep = valid ? 1 : 0;
  int ok = i == 0 ? 1 : (valid && node_tok[i] == pred[p]) ? 1 : 0;
#pragma unroll
  for (int k = 0; k < 5; ++k) {
    const int src = up < 0 ? i : up;
    const int up2 = __shfl(up, src), dep2 = __shfl(dep, src), ok2 = __shfl(ok, src);
    if (up >= 0) {
      ok &= ok2;
      dep += dep2;
      up = up2;
    }
  }
  // deepest accepted node, lowest index on ties: max of (depth, 63 - index)
  uint32_t key = node && ok ? ((uint32_t)dep << 8) | (uint32_t)(63 - i) : 0u;
  key = max(key, xor_lane<1>(key));
  key = max(key, xor_lane<2>(key));
  key = max(key, xor_lane<4>(key));
  key = max(key, xor_lane<8>(key));
  key = max(key, xor_lane<16>(key));
  key = max(key, xor_lane<32>(key));
  const int best = 63 - (int)(key & 0xFFu), n = (int)(key >> 8);
  // path[d] (the ancestor of best at depth d) in lane d, walking up from best
  int path = -1;
  for (int d = n, j = best; d >= 0; --d) {
    if (i == d) path = j;
    j = __shfl(p, j);
  }
  const int next = __shfl(path, (i + 1) & 63);  // path[i + 1]
  const int64_t t = pred[best];
  const int64_t base = *o.pos;
  if (node) {
    o.tokens[i] = i < n ? node_tok[next] : (i == n ? t : -1);
    o.commit[i] = i <= n ? path : -1;
  }
  if (i == 0) {
    *o.n_accepted = n;
    *o.tok = t;
    *o.pos = base + n + 1;
    *o.slot = best;
  }
}

// ------------------------------------------------------------------ argmax kernel (greedy, tree)

}  // namespace tr
