// On-device accept/commit of the speculative verify step, for gfx950.
//
// Every kernel splits each vocabulary row into chunks handled by separate workgroups and
// finishes with "last arriver" reductions: each workgroup publishes its partial result to the
// caller's workspace with agent-scope stores, then increments a per-row counter; the workgroup
// that brings the counter to its total reduces the row (and, one level up, the last row
// finishes the accept). Counters are reset by the workgroup that consumes them, so a zero-filled
// workspace stays valid across calls and graph replays, and one launch does the whole job.
//
// Arithmetic is fixed so that the CPU oracle (oracle/accept.py) reproduces it bit for bit:
//   * texp(): Cody-Waite reduction with ln2 split hi/lo, degree-7 Taylor polynomial of e^r in
//     Horner form, 2^n through the exponent field; x < -80 -> 0. Constants are fp32 bit
//     patterns. The file is compiled with -ffp-contract=off and uses explicitly rounded
//     operations, so every step is one fp32 rounding.
//   * sums over the 64 sampling candidates are sequential in rank order;
//   * sums over a vocabulary row are blocked: sequential over runs of 16 elements, over the 64
//     runs of a 1024-element chunk, then over chunks.
//   * ties: argmax takes the first index; the top-64 candidates are ordered by value
//     descending, then index ascending.
// Logits are bf16; NaN logits are not supported.
#include "accept_common.h"

namespace tr {

// ------------------------------------------------------------------ shared helpers

constexpr int kCand = 64;          // sampling candidates (tokenrush/sample.py:12)
constexpr int kTopChunk = 4096;    // elements per workgroup in the top-64 kernel
// elements per workgroup in the argmax kernel: 4096 up to 8 rows, 16384 above (about 500
// workgroups either way: enough to stream the logits, few per-row handshakes)
constexpr int kArgChunkSmall = 4096, kArgChunkLarge = 16384;
constexpr int kRun = 16, kChunk = 1024;
constexpr int kMaxChunks = 256;    // 1024-element chunks per row: V <= 262144
constexpr int kCntStride = 64;     // ints between workspace counters (one 256-byte line each)

// All threads of the block copy n workspace values into LDS with independent agent-scope loads
// (a serial chain of such loads would cost a memory round trip each).
template <typename T>
__device__ __forceinline__ void ws_gather(const T* src, int n, T* dst) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) dst[i] = ws_ld(src + i);
  __syncthreads();
}

// The same fixed left-to-right fp32 chains, run by a whole wave over values held in registers:
// element j of the sequence is lane j % 64 of r[j / 64]. v_readlane brings each element to a
// scalar register in index order, so every lane computes exactly the sequential result, without
// a memory or LDS round trip per element (a lane-0 loop that waits for an LDS load per element
// costs ~70 ns per element; wave_seq_prefix below loads its blocks ahead).
// Callers pass zeros past the sequence's end: the chains are over non-negative values, to which
// adding +0 changes nothing, so no per-element bound check (a divergent branch) is needed.
__device__ __forceinline__ float lane_val(float v, int i) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
}
// The compiler would hoist every v_readlane of a chain ahead of its adds and run out of scalar
// registers (spills); an empty asm that "writes" the value register every 16 elements keeps the
// readlanes of one block after the previous block's adds.
template <int R>
__device__ __forceinline__ float wave_seq_sum(const float (&r)[R]) {
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    float x = r[k];
#pragma unroll
    for (int i = 0; i < 64; ++i) {
      if ((i & 15) == 0) asm volatile("" : "+v"(x), "+v"(s));
      s = __fadd_rn(s, lane_val(x, i));
    }
  }
  return s;
}
// Running sums acc + x_0 + ... + x_j (left to right): lane i of pre[k] gets element 64 k + i's.
// Lane 0 alone runs the chain over a copy in LDS (lds: 64 R floats, 16-byte aligned, private to
// the wave): the values go to LDS, lane 0 reads them back in blocks and runs the chain as plain
// dependent adds, writing each running sum in place, and every lane reads its own. (Chains on
// v_readlane with each sum selected into its lane cost about twice as much per element.)
template <int R>
__device__ __forceinline__ void wave_seq_prefix(const float (&r)[R], float acc, float (&pre)[R], float* lds) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < R; ++k) lds[64 * k + lane] = r[k];
  asm volatile("" ::: "memory");
  if (lane == 0) {
    // 32 values a block; the next block's loads are issued (and pinned by the clobber) before
    // the current block's adds, so that they are in flight meanwhile
    float4* b = (float4*)lds;
    constexpr int NB = 8, NQ = 16 * R;
    float4 cur[NB], nxt[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) cur[t] = b[t];
#pragma unroll
    for (int q = 0; q < NQ; q += NB) {
      if (q + NB < NQ) {
#pragma unroll
        for (int t = 0; t < NB; ++t) nxt[t] = b[q + NB + t];
      }
      asm volatile("" ::: "memory");
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        acc = __fadd_rn(acc, cur[t].x); cur[t].x = acc;
        acc = __fadd_rn(acc, cur[t].y); cur[t].y = acc;
        acc = __fadd_rn(acc, cur[t].z); cur[t].z = acc;
        acc = __fadd_rn(acc, cur[t].w); cur[t].w = acc;
      }
#pragma unroll
      for (int t = 0; t < NB; ++t) b[q + t] = cur[t];
#pragma unroll
      for (int t = 0; t < NB; ++t) cur[t] = nxt[t];
    }
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int k = 0; k < R; ++k) pre[k] = lds[64 * k + lane];
  asm volatile("" ::: "memory");
}
// Given the running sums pre of r from acc: the first element whose running sum exceeds target,
// else the last positive element (-1 if none); *base gets the running sum before it. Uniform.
template <int R>
__device__ __forceinline__ int wave_seq_choose(const float (&r)[R], const float (&pre)[R], float acc, float target, float* base) {
  int chosen = -1;
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const unsigned long long m = __ballot(pre[k] > target);
    if (chosen < 0 && m) chosen = 64 * k + __ffsll((long long)m) - 1;
  }
#pragma unroll
  for (int k = R - 1; k >= 0; --k) {
    const unsigned long long m = __ballot(r[k] > 0.f);
    if (chosen < 0 && m) chosen = 64 * k + 63 - __clzll((long long)m);
  }
  chosen = __builtin_amdgcn_readfirstlane(chosen);
  float b = acc;
  const int pj = chosen - 1;
  if (pj >= 0) {
    float sel = pre[0];
#pragma unroll
    for (int k = 1; k < R; ++k) sel = (pj >> 6) == k ? pre[k] : sel;
    b = lane_val(sel, pj & 63);
  }
  *base = b;
  return chosen;
}
// The sequential inverse-CDF step over r from acc (wave_seq_choose of wave_seq_prefix).
template <int R>
__device__ __forceinline__ int wave_seq_search(const float (&r)[R], float acc, float target, float* base, float* lds) {
  float pre[R];
  wave_seq_prefix(r, acc, pre, lds);
  return wave_seq_choose(r, pre, acc, target, base);
}

// Block-wide exclusive prefix sum of one int per thread (blockDim.x <= 1024), plus the total.
__device__ int block_exclusive_scan(int v, int* total) {
  __shared__ int wsum[16];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wsum[wid] = x;
  __syncthreads();
  int base = 0, tot = 0;
  for (int w = 0; w < nw; ++w) {
    if (w < wid) base += wsum[w];
    tot += wsum[w];
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

// e^x for x <= 0 (see the file comment).
__device__ float texp(float x) {
  if (!(x >= -80.f)) return 0.f;
  const float kLog2e = __uint_as_float(0x3FB8AA3Bu), kLn2Hi = __uint_as_float(0x3F317200u),
              kLn2Lo = __uint_as_float(0x35BFBE8Eu);
  const float c[8] = {__uint_as_float(0x3F800000u), __uint_as_float(0x3F800000u), __uint_as_float(0x3F000000u),
                      __uint_as_float(0x3E2AAAABu), __uint_as_float(0x3D2AAAABu), __uint_as_float(0x3C088889u),
                      __uint_as_float(0x3AB60B61u), __uint_as_float(0x39500D01u)};
  const float t = __fmul_rn(x, kLog2e);
  const float n = rintf(t);
  float r = __fsub_rn(x, __fmul_rn(n, kLn2Hi));
  r = __fsub_rn(r, __fmul_rn(n, kLn2Lo));
  float p = c[7];
#pragma unroll
  for (int k = 6; k >= 0; --k) p = __fadd_rn(__fmul_rn(p, r), c[k]);
  int ni = (int)n;
  ni = ni < -126 ? -126 : (ni > 127 ? 127 : ni);
  return __fmul_rn(p, __int_as_float((ni + 127) << 23));
}

// One compare-exchange stage of a 64-lane bitonic sort (final order descending): partner lane
// tid ^ STRIDE, direction from the SIZE-block (cross-lane moves on the VALU, xor_lane64).
template <int SIZE, int STRIDE>
__device__ __forceinline__ uint64_t sort_step(uint64_t key, int tid) {
  const uint64_t other = xor_lane64<STRIDE>(key);
  const bool desc = (tid & SIZE) == 0;
  const bool lower = (tid & STRIDE) == 0;
  const bool keep_max = desc == lower;
  return keep_max ? (other > key ? other : key) : (other < key ? other : key);
}

// Top-64 of up to 256 * E items held E per thread, items of thread t preceding those of
// thread t+1 in index order. Keys are ord16 values (0 = padding). Result in LDS out_k/out_i
// (64 entries, value descending then index ascending); needs blockDim.x == 256.
template <int E>
__device__ void select_top64(const uint32_t (&k16)[E], const uint32_t (&idx)[E], uint32_t* out_k, uint32_t* out_i) {
  __shared__ int hist[256];
  __shared__ uint32_t sel_k[kCand], sel_i[kCand];
  __shared__ uint32_t s_bin, s_above;
  const int tid = threadIdx.x;
  uint32_t prefix = 0, prefix_mask = 0;
  int remaining = kCand;
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = pass == 0 ? 8 : 0;
    hist[tid] = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < E; ++e)
      if ((k16[e] & prefix_mask) == prefix) atomicAdd(&hist[(k16[e] >> shift) & 0xFF], 1);
    __syncthreads();
    if (tid < 64) {
      // lane l owns bins 4l..4l+3; find the bin where the count from the top reaches `remaining`
      const int h0 = hist[4 * tid], h1 = hist[4 * tid + 1], h2 = hist[4 * tid + 2], h3 = hist[4 * tid + 3];
      const int s = h0 + h1 + h2 + h3;
      int above = s;  // inclusive suffix sum over lanes >= tid
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_down(above, o);
        if (tid + o < 64) above += y;
      }
      const int strictly_above = above - s;  // items in bins of higher lanes
      if (strictly_above < remaining && above >= remaining) {
        int acc = strictly_above, b = 3;
        const int hh[4] = {h0, h1, h2, h3};
        while (b > 0 && acc + hh[b] < remaining) acc += hh[b--];
        s_bin = 4 * tid + b;
        s_above = acc;
      }
      if (tid == 0 && above < remaining) {  // fewer items than 64: take everything
        s_bin = 0;
        s_above = above - h0;
      }
    }
    __syncthreads();
    prefix |= s_bin << shift;
    prefix_mask |= 0xFFu << shift;
    remaining -= s_above;
    __syncthreads();
  }
  const uint32_t T = prefix;
  // ties at T are taken in index order: rank them with a block scan
  int ties = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) ties += k16[e] == T;
  int tot;
  int tie_rank = block_exclusive_scan(ties, &tot);
  int nsel = 0;
  bool take[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    take[e] = k16[e] > T || (k16[e] == T && tie_rank < remaining);
    if (k16[e] == T) ++tie_rank;
    nsel += take[e];
  }
  int pos = block_exclusive_scan(nsel, &tot);
#pragma unroll
  for (int e = 0; e < E; ++e)
    if (take[e] && pos < kCand) {
      sel_k[pos] = k16[e];
      sel_i[pos] = idx[e];
      ++pos;
    }
  if (tid >= tot && tid < kCand) {  // fewer than 64 items
    sel_k[tid] = 0;
    sel_i[tid] = 0xFFFFFFFFu;
  }
  __syncthreads();
  if (tid < 64) {
    // bitonic sort of 64 (value desc, index asc) keys across the lanes of wave 0
    uint64_t key = vkey(sel_k[tid], sel_i[tid]);
    key = sort_step<2, 1>(key, tid);
    key = sort_step<4, 2>(key, tid);
    key = sort_step<4, 1>(key, tid);
    key = sort_step<8, 4>(key, tid);
    key = sort_step<8, 2>(key, tid);
    key = sort_step<8, 1>(key, tid);
    key = sort_step<16, 8>(key, tid);
    key = sort_step<16, 4>(key, tid);
    key = sort_step<16, 2>(key, tid);
    key = sort_step<16, 1>(key, tid);
    key = sort_step<32, 16>(key, tid);
    key = sort_step<32, 8>(key, tid);
    key = sort_step<32, 4>(key, tid);
    key = sort_step<32, 2>(key, tid);
    key = sort_step<32, 1>(key, tid);
    key = sort_step<64, 32>(key, tid);
    key = sort_step<64, 16>(key, tid);
    key = sort_step<64, 8>(key, tid);
    key = sort_step<64, 4>(key, tid);
    key = sort_step<64, 2>(key, tid);
    key = sort_step<64, 1>(key, tid);
    out_k[tid] = (uint32_t)(key >> 32);
    out_i[tid] = vkey_idx(key);
  }
  __syncthreads();
}


// Helpers of the threshold top-64 (sample_kernel). Every item's key is unique (value, then index),
// so ranks and the resulting list do not depend on the order candidates were gathered in.

// The largest v with at least K of the wave's 64 * R keys >= v (bit by bit from the top):
// uniform over the wave.
template <int K, int R>
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&kv)[R]) {
  uint32_t v = 0;
#pragma unroll
  for (int b = 15; b >= 0; --b) {
    const uint32_t c = v | (1u << b);
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) cnt += __popcll(__ballot(kv[r] >= c));
    v = cnt >= K ? c : v;
  }
  return v;
}

// The top 64 of n <= kTopCap candidate keys (vkey()s) in LDS, by rank: thread t compares
// candidate t % kTopCap with one half of the n (rounded up to 32) slots, the halves' counts meet
// in rank[] (zeroed by the caller), and the candidates of rank < 64 land at their rank. 256
// threads.
constexpr int kTopCap = 128;
__device__ void lds_rank_top64(const uint64_t* kk, int n, int* rank, uint32_t* out_k, uint32_t* out_i) {
  const int tid = threadIdx.x, c = tid & (kTopCap - 1), half = tid >> 7;
  if (c < n) {
    const uint64_t key = kk[c];
    int r0 = 0, r1 = 0, r2 = 0, r3 = 0;
    const int h = ((n + 31) >> 5) << 4;  // half of n rounded up to 32: 2 h <= kTopCap
    const int j0 = half * h;
    for (int j = 0; j < h; j += 16) {  // slots past n hold 0: below every key
      uint64_t v[16];  // 16 LDS reads in flight per round trip
#pragma unroll
      for (int q = 0; q < 16; ++q) v[q] = kk[j0 + j + q];
#pragma unroll
      for (int q = 0; q < 16; q += 4) {
        r0 += v[q] > key;
        r1 += v[q + 1] > key;
        r2 += v[q + 2] > key;
        r3 += v[q + 3] > key;
      }
    }
    atomicAdd(&rank[c], (r0 + r1) + (r2 + r3));
  }
  __syncthreads();
  if (tid < n) {
    const int r = rank[tid];
    if (r < kCand) {
      out_k[r] = (uint32_t)(kk[tid] >> 32);
      out_i[r] = vkey_idx(kk[tid]);
    }
  }
  __syncthreads();
}

// Appends this thread's items with keys >= tau to kk[] as vkey()s. Each thread counts its items;
// the exclusive prefix of the counts over the wave comes from one ballot per count bit, and one LDS atomic per wave places the wave. Returns the total after a
// barrier (uniform); nothing is written when it exceeds kTopCap.
template <int E>
__device__ int lds_append_keys(const uint32_t (&k16)[E], const uint32_t (&idx)[E], uint32_t tau, uint64_t* kk, int* cnt) {
  static_assert(E < 64, "per-thread counts must fit six bits");
  constexpr int kBits = E < 32 ? 5 : 6;
  const int lane = threadIdx.x & 63;
  int c = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) c += k16[e] >= tau ? 1 : 0;
  int pre = 0, wtot = 0;
#pragma unroll
  for (int b = 0; b < kBits; ++b) {
    const unsigned long long m = __ballot((c >> b) & 1);
    pre += (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << b;
    wtot += __popcll(m) << b;
  }
  int base = 0;
  if (lane == 0 && wtot) base = atomicAdd(cnt, wtot);
  base = __builtin_amdgcn_readfirstlane(base);
  __syncthreads();
  const int tot = *cnt;
  if (tot <= kTopCap) {
    int pos = base + pre;
#pragma unroll
    for (int e = 0; e < E; ++e)
      if (k16[e] >= tau) kk[pos++] = vkey(k16[e], idx[e]);
  }
  __syncthreads();
  return tot;
}

// Top-64 of a chunk by a threshold (the fast path of sample_kernel's per-chunk select). tau =
// the 64th largest of the 128 maxima of thread pairs bounds the chunk's 64th largest key from
// below: the 64 pairs whose maxima reach it hold 64 items >= tau. Items >= tau (typically ~89 of
// 4096 for continuous data, at most 115 in 2000 simulated chunks) are ranked; more than kTopCap of
// them (heavy ties, padding) take select_top64 instead. Both give the same list: the exact top 64, value descending then index ascending.
template <int E>
__device__ void select_top64_thr(const uint32_t (&k16)[E], const uint32_t (&idx)[E], uint32_t* out_k, uint32_t* out_i) {
  __shared__ uint64_t kk[kTopCap];
  __shared__ int rank[kTopCap];
  __shared__ uint32_t tmax[256];
  __shared__ uint32_t s_tau;
  __shared__ int s_cnt;
  const int tid = threadIdx.x, lane = tid & 63;
  uint32_t m = 0;
#pragma unroll
  for (int e = 0; e < E; ++e) m = k16[e] > m ? k16[e] : m;
  tmax[tid] = m;
  if (tid < kTopCap) {
    kk[tid] = 0ull;
    rank[tid] = 0;
  }
  if (tid == 0) s_cnt = 0;
  __syncthreads();
  if (tid < 64) {
    // the 64th largest of the 128 maxima of thread pairs (t, t + 128): still 64 items >= it, at
    // half the ballots of the 256 thread maxima (~89 candidates instead of ~74 for continuous data)
    const uint32_t mv[2] = {max(tmax[lane], tmax[128 + lane]), max(tmax[64 + lane], tmax[192 + lane])};
    const uint32_t v = wave_kth<kCand>(mv);
    if (lane == 0) s_tau = v;
  }
  __syncthreads();
  const int tot = lds_append_keys(k16, idx, s_tau, kk, &s_cnt);
  if (tot > kTopCap) {  // uniform
    select_top64<E>(k16, idx, out_k, out_i);
    return;
  }
  lds_rank_top64(kk, tot, rank, out_k, out_i);
}

// Wave-wide merge of two descending 64-key lists, one key per lane: lane i keeps the larger of
// a[i] and b[63 - i] (the top 64 of the union, as a bitonic sequence), then a bitonic merge
// sorts it descending. Keys are vkey()s: value descending, index ascending.
template <int S>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t key, int lane) {
  const uint64_t other = xor_lane64<S>(key);
  const bool lower = (lane & S) == 0;
  return lower ? (other > key ? other : key) : (other < key ? other : key);
}
__device__ __forceinline__ uint64_t bitonic_sort_desc(uint64_t key, int lane) {
  key = bitonic_step<32>(key, lane);
  key = bitonic_step<16>(key, lane);
  key = bitonic_step<8>(key, lane);
  key = bitonic_step<4>(key, lane);
  key = bitonic_step<2>(key, lane);
  return bitonic_step<1>(key, lane);
}
__device__ __forceinline__ uint64_t merge_top64(uint64_t a, uint64_t b_rev, int lane) {
  return bitonic_sort_desc(a > b_rev ? a : b_rev, lane);
}

// Top 64 (descending) of n <= 16 * waves sorted 64-key lists in the workspace (list c at
// src + 128 c: 64 (value key, index) pairs), merged by the block's waves; result in LDS
// out_k / out_i.
__device__ void merge_lists_top64(const uint32_t* src, int n, uint32_t* out_k, uint32_t* out_i) {
  constexpr int kPerWave = 16;  // lists per wave: n <= 64 with 4 waves
  __shared__ uint64_t wres[16][kCand];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // every list of this wave is loaded before any merge: independent loads, one round trip. The
  // loads are unconditional (lists past n re-read list n - 1 and are dropped afterwards): an
  // agent-scope load under a condition cannot be speculated, and the branch around each one
  // made the compiler wait for it before the next.
  uint32_t kv[kPerWave], iv[kPerWave];
#pragma unroll
  for (int j = 0; j < kPerWave; ++j) {
    const int c = wid + j * nw;
    const int cc = c < n ? c : n - 1;
    const uint64_t* l = (const uint64_t*)(src + (size_t)cc * kCand * 2 + 2 * (kCand - 1 - lane));  // reversed: ascending
    const uint64_t v = ws_ld(l);  // (key16, index) pair
    kv[j] = c < n ? (uint32_t)v : 0u;
    iv[j] = c < n ? (uint32_t)(v >> 32) : 0xFFFFFFFFu;
  }
  // merging a padding list (all keys minimal) leaves acc unchanged, so every merge runs: no
  // branch, no wait for the loads of lists that are not merged yet
  uint64_t acc = bitonic_sort_desc(vkey(kv[0], iv[0]), lane);
#pragma unroll
  for (int j = 1; j < kPerWave; ++j) acc = merge_top64(acc, vkey(kv[j], iv[j]), lane);
  wres[wid][lane] = acc;
  __syncthreads();
  if (wid == 0) {
    for (int w = 1; w < nw; ++w) acc = merge_top64(acc, wres[w][kCand - 1 - lane], lane);
    out_k[lane] = (uint32_t)(acc >> 32);
    out_i[lane] = vkey_idx(acc);
  }
  __syncthreads();
}

// The row's top 64 from n <= 64 sorted chunk lists (as merge_lists_top64), by a threshold: tau =
// the 64th largest of the maxima of pairs of the lists' first four keys bounds the row's 64th
// largest from below; the entries >= tau (a prefix of each list) are ranked as in
// select_top64_thr. More than kTopCap of them take merge_lists_top64 instead; both give the same
// list. Load j of wave w brings list 4 j + w, rank `lane` (one list per load: 4 cache lines,
// where a list per lane touched 64), all loads issued at once; the lists' first four keys
// meet in LDS for tau.
__device__ void merge_lists_top64_thr(const uint32_t* src, int n, uint32_t* out_k, uint32_t* out_i) {
  constexpr int kR = 16;
  __shared__ uint64_t kk[kTopCap];
  __shared__ int rank[kTopCap];
  __shared__ uint32_t heads[4 * kCand];
  __shared__ uint32_t s_tau;
  __shared__ int s_cnt;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint32_t kv[kR], iv[kR];
#pragma unroll
  for (int j = 0; j < kR; ++j) {
    const int c = 4 * j + wid;  // list
    const uint64_t v = ws_ld((const uint64_t*)(src + (size_t)(c < n ? c : n - 1) * kCand * 2 + 2 * lane));
    kv[j] = c < n ? (uint32_t)v : 0u;
    iv[j] = (uint32_t)(v >> 32);
  }
  if (tid < kTopCap) {
    kk[tid] = 0ull;
    rank[tid] = 0;
  }
  if (tid == 0) s_cnt = 0;
  if (lane < 4) {
#pragma unroll
    for (int j = 0; j < kR; ++j) heads[4 * (4 * j + wid) + lane] = kv[j];
  }
  __syncthreads();
  if (wid == 0) {
    // the 64th largest of the maxima of head pairs: 64 list items >= it (as in select_top64_thr)
    const uint32_t head[2] = {max(heads[lane], heads[128 + lane]), max(heads[64 + lane], heads[192 + lane])};
    const uint32_t v = wave_kth<kCand>(head);
    if (lane == 0) s_tau = v;
  }
  __syncthreads();
  const int tot = lds_append_keys(kv, iv, s_tau, kk, &s_cnt);
  if (tot > kTopCap) {  // uniform
    merge_lists_top64(src, n, out_k, out_i);
    return;
  }
  lds_rank_top64(kk, tot, rank, out_k, out_i);
}

// ------------------------------------------------------------------ accept outputs

enum { FIN_NONE = 0, FIN_CHAIN = 1, FIN_TREE = 2 };

struct ArgmaxArgs {
  const uint16_t* logits;  // bf16 [M, V]
  int M, V, nch, fin;
  const int64_t* spec;     // chain: committed + drafts [M]; tree: node tokens [M]
  const int32_t* parent;   // tree: [M]
  uint64_t* keys;          // ws [M * nch]
  int64_t* preds;          // ws [M]
  int* cnt_rows;           // ws [M]
  int* cnt_all;            // ws [1]
  AcceptOut o;
};

template <int kArgChunk>
__global__ __launch_bounds__(256) void argmax_kernel(ArgmaxArgs a) {
  const int row = blockIdx.x / a.nch, ch = blockIdx.x % a.nch;
  const int beg = ch * kArgChunk;
  const uint16_t* lg = a.logits + (size_t)row * a.V;
  uint64_t best = 0;
  if ((a.V & 7) == 0) {
    // 16-byte loads: thread t reads elements beg + 8 t + 2048 h + (0..7), h = 0..7, all issued at
    // once (past the row end: the row's last 8 elements again, not counted)
    constexpr int kH = kArgChunk / 2048;
    uint4 v[kH];
#pragma unroll
    for (int h = 0; h < kH; ++h) {
      const int i0 = beg + h * 2048 + threadIdx.x * 8;
      v[h] = *(const uint4*)(lg + min(i0, a.V - 8));
    }
#pragma unroll
    for (int h = 0; h < kH; ++h) {
      const int i0 = beg + h * 2048 + threadIdx.x * 8;
      const uint32_t w[4] = {v[h].x, v[h].y, v[h].z, v[h].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint64_t k = vkey(ord16((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu), i0 + e);
        best = (i0 < a.V && k > best) ? k : best;
      }
    }
  } else {
    for (int i = beg + threadIdx.x; i < min(a.V, beg + kArgChunk); i += blockDim.x) {
      const uint64_t k = vkey(ord16(lg[i]), i);
      best = k > best ? k : best;
    }
  }
  best = wave_max_u64(best);
  __shared__ uint64_t wmax[4];
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) best = wmax[w] > best ? wmax[w] : best;
    ws_st(a.keys + blockIdx.x, best);
  }
  if (!arrive_last(a.cnt_rows + row * kCntStride, a.nch)) return;
  if (threadIdx.x < 64) {
    uint64_t b = 0;
    for (int c = threadIdx.x; c < a.nch; c += 64) {
      const uint64_t k = ws_ld(a.keys + (size_t)row * a.nch + c);
      b = k > b ? k : b;
    }
    b = wave_max_u64(b);
    if (threadIdx.x == 0) {
      const int64_t idx = vkey_idx(b);
      if (a.o.pred) a.o.pred[row] = idx;
      ws_st(a.preds + row, idx);
    }
  }
  if (!arrive_last(a.cnt_all, a.M)) return;
  if (a.fin == FIN_NONE) return;
  __shared__ int64_t pred[32], spec[32];
  __shared__ int32_t parent[32];
  if (threadIdx.x < a.M) {
    spec[threadIdx.x] = a.spec[threadIdx.x];
    if (a.fin == FIN_TREE) parent[threadIdx.x] = a.parent[threadIdx.x];
  }
  ws_gather(a.preds, a.M, pred);
  if (a.fin == FIN_CHAIN) {
    if (threadIdx.x < 64) finish_chain(pred, spec, a.M, a.o);
  } else if (threadIdx.x < 64) {
    finish_tree(pred, spec, parent, a.M, a.o);
  }
}

// ------------------------------------------------------------------ sample kernel (sample.py:30-51)

struct SampleArgs {
  const uint16_t* logits;
  int M, V, nch, fin;
  const float* temperature;  // [1] device (0 = greedy)
  const float* top_p;        // [1]
  const int64_t* top_k;      // [1]
  const float* u;            // [M] uniforms in [0, 1)
  const int64_t* spec;       // chain: committed + drafts [M]
  uint32_t* cand;            // ws [M * nch * 64 * 2] (key16, index)
  int64_t* preds;            // ws [M]
  int* cnt_rows;
  int* cnt_all;
  int64_t* out;              // [M] sampled tokens (may be null)
  AcceptOut o;
};

// One row's pick from its sorted top-64 (value desc, index asc), by wave 0: elementwise steps
// on lane i = rank i, the running sums in rank order by wave chains (the file comment's fixed
// order). Returns the token in every lane of wave 0.
__device__ int64_t sample_pick(const uint32_t* tk, const uint32_t* ti, float T, float top_p, int64_t top_k, float u) {
  const int i = threadIdx.x;  // 0..63
  if (!(T > 0.f)) return ti[0];
  const float temp = T > __uint_as_float(0x358637BDu) ? T : __uint_as_float(0x358637BDu);
  const float sv = __fdiv_rn(bf16_bits_to_f32(unord16(tk[i])), temp);
  const float e = texp(__fsub_rn(sv, lane_val(sv, 0)));
  const float er[1] = {e};
  const float p = __fdiv_rn(e, wave_seq_sum(er));
  // cumulative sums in rank order; lane i keeps the sum through rank i
  __shared__ __align__(16) float cum_s[64];
  const float pr[1] = {p};
  float cum[1];
  wave_seq_prefix(pr, 0.f, cum, cum_s);
  const bool keep = __fsub_rn(cum[0], p) < top_p && i < top_k;
  // The kept ranks are a prefix: p is sorted descending and fl(c + p) >= c, so cum - p never
  // decreases from one rank to the next, nor does its rounding. The running sums of the kept p
  // are therefore the first running sums bit for bit, and past the last kept rank they stay at
  // its value (adding zeros): no second sequential pass.
  const unsigned long long kept = __ballot(keep);
  const float last = kept ? lane_val(cum[0], 63 - __clzll((long long)kept)) : 0.f;
  const float target = __fmul_rn(u, last);
  const float mycum2 = keep ? cum[0] : last;
  const unsigned long long below = __ballot(mycum2 < target);
  int pick = __popcll(below);
  if (pick > kCand - 1) pick = kCand - 1;
  return ti[pick];
}

__global__ __launch_bounds__(256) void sample_kernel(SampleArgs a) {
  constexpr int E = kTopChunk / 256;
  __shared__ uint32_t tk[kCand], ti[kCand];
  const int row = blockIdx.x / a.nch, ch = blockIdx.x % a.nch;
  const int beg = ch * kTopChunk;
  const uint16_t* lg = a.logits + (size_t)row * a.V;
  uint32_t k16[E], idx[E];
  const int i0 = beg + threadIdx.x * E;
  if ((a.V & 7) == 0 && i0 + E <= a.V) {
#pragma unroll
    for (int h = 0; h < E / 8; ++h) {
      const uint4 v = *(const uint4*)(lg + i0 + 8 * h);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        idx[8 * h + e] = i0 + 8 * h + e;
        k16[8 * h + e] = ord16((w[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int i = i0 + e;
      idx[e] = i;
      k16[e] = i < a.V ? ord16(lg[i]) : 0u;
    }
  }
  select_top64_thr<E>(k16, idx, tk, ti);
  uint32_t* mine = a.cand + ((size_t)row * a.nch + ch) * kCand * 2;
  if (threadIdx.x < kCand) {
    ws_st(mine + 2 * threadIdx.x, tk[threadIdx.x]);
    ws_st(mine + 2 * threadIdx.x + 1, ti[threadIdx.x]);
  }
  if (!arrive_last(a.cnt_rows + row * kCntStride, a.nch)) return;
  merge_lists_top64_thr(a.cand + (size_t)row * a.nch * kCand * 2, a.nch, tk, ti);
  if (threadIdx.x < 64) {
    const int64_t t = sample_pick(tk, ti, *a.temperature, *a.top_p, *a.top_k, a.u[row]);
    if (threadIdx.x == 0) {
      if (a.out) a.out[row] = t;
      ws_st(a.preds + row, t);
    }
  }
  if (!arrive_last(a.cnt_all, a.M)) return;
  if (a.fin != FIN_CHAIN) return;
  __shared__ int64_t pred[32], spec[32];
  if (threadIdx.x < a.M) spec[threadIdx.x] = a.spec[threadIdx.x];
  ws_gather(a.preds, a.M, pred);
  if (a.o.pred && threadIdx.x < a.M) a.o.pred[threadIdx.x] = pred[threadIdx.x];
  if (threadIdx.x < 64) finish_chain(pred, spec, a.M, a.o);
}

// ------------------------------------------------------------------ residual rejection sampling

// Exponentials are taken per 1024-element chunk: with m_c the chunk's maximum and M the row's,
// a = texp(l - m_c), f_c = texp(m_c - M), e = fl(a f_c) (0 below the smallest normal), and
// Z = the group-blocked sum of fl(f_c A_c), A_c the chunk's blocked sum of a. So no pass waits
// for a row maximum; p = fl(e fl(1 / Z)). Phase 2: per (row, chunk) m_c and A_c, and a(d_i), q_i(d_i), m_c(d_i)
// kept by the chunk holding draft d_i; the row's last workgroup takes M and Z. Phase 3: the
// accept tests u_i q_i(d_i) < e_i(d_i) / Z_i (in every wave), then the draw from row n.
struct ResidualArgs {
  const uint16_t* logits;  // [K+1, V]
  const float* q;          // [K, V]
  const int64_t* spec;     // committed + K drafts [K+1]
  const float* u;          // [K+1]
  int M, V, nch;           // M = K + 1 rows, nch = 1024-chunks per row
  float* A;                // ws [M * nch]: chunk sums of a (phase 2)
  float* mc;               // ws [M * nch]: chunk maxima (phase 2)
  float* chunk_sum;        // ws [nch]: phase 3's chunk sums of r
  float* rowmax;           // ws [M]
  float* Z;                // ws [M]
  float* a_draft;          // ws [M]: a(d_i), q_i(d_i) and m_c(d_i), stored by the chunk holding d_i
  float* q_draft;
  float* m_draft;
  int* cnt_rows;
  int* cnt_all;
  AcceptOut o;
};

constexpr float kFltMin = 1.17549435e-38f;  // smallest normal fp32: products below it count as 0

// Wave maxima of an unsigned key and of a float (DPP / permlane exchanges).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  uint32_t w;
  w = xor_lane<32>(v); v = w > v ? w : v;
  w = xor_lane<16>(v); v = w > v ? w : v;
  w = xor_lane<8>(v); v = w > v ? w : v;
  w = xor_lane<4>(v); v = w > v ? w : v;
  w = xor_lane<2>(v); v = w > v ? w : v;
  w = xor_lane<1>(v); v = w > v ? w : v;
  return v;
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __uint_as_float(xor_lane<32>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(xor_lane<16>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(xor_lane<8>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(xor_lane<4>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(xor_lane<2>(__float_as_uint(v))));
  v = fmaxf(v, __uint_as_float(xor_lane<1>(__float_as_uint(v))));
  return v;
}

// This lane's run (16 elements) of chunk ch of row `row`: logits bits as loaded (two per word,
// unpacked only where used, so that a load can stay in flight), and q (residual only).
struct RunData {
  uint32_t lw[kRun / 2];
  float qv[kRun];
};
template <int MODE>  // 0: e, 1: residual, 2: p
__device__ __forceinline__ void run_load(const ResidualArgs& a, int row, int ch, int lane, RunData& d) {
  const uint16_t* lg = a.logits + (size_t)row * a.V;
  const float* qr = a.q + (size_t)row * a.V;
  const int i0 = ch * kChunk + lane * kRun;
  float (&qv)[kRun] = d.qv;
  if ((a.V & 7) == 0 && i0 + kRun <= a.V) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint4 v = *(const uint4*)(lg + i0 + 8 * h);
      d.lw[4 * h] = v.x;
      d.lw[4 * h + 1] = v.y;
      d.lw[4 * h + 2] = v.z;
      d.lw[4 * h + 3] = v.w;
    }
    if (MODE == 1) {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float4 v = *(const float4*)(qr + i0 + 4 * h);
        qv[4 * h] = v.x;
        qv[4 * h + 1] = v.y;
        qv[4 * h + 2] = v.z;
        qv[4 * h + 3] = v.w;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < kRun; ++e) {
      const uint32_t b = i0 + e < a.V ? lg[i0 + e] : 0u;
      d.lw[e >> 1] = (e & 1) ? (d.lw[e >> 1] | (b << 16)) : b;
      if (MODE == 1) qv[e] = i0 + e < a.V ? qr[i0 + e] : 0.f;
    }
  }
}
// The run's values from its loaded data, m = the chunk's maximum and f its factor f_c:
// r = p - q clamped at 0 (residual), or p (bonus), p = fl(e fl(1 / Z)), or a (phase 2; f and
// invZ unused). Returns the sequential run sum.
// The chunk's maximum logit (bf16 value as fp32) from the run's loaded words: the ordered bf16
// keys of the valid elements, then the wave. Phases 2 and 3 take it from the same words.
__device__ __forceinline__ float chunk_max(const ResidualArgs& a, int ch, int lane, const RunData& d) {
  const int i0 = ch * kChunk + lane * kRun;
  uint32_t km = 0;
#pragma unroll
  for (int e = 0; e < kRun; ++e) {
    const uint32_t k = ord16((d.lw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
    km = (i0 + e < a.V && k > km) ? k : km;
  }
  return bf16_bits_to_f32(unord16(wave_max_u32(km)));
}

template <int MODE>
__device__ __forceinline__ float r_value(const ResidualArgs& a, int i0, float mx, float f, float invZ, const RunData& d, int e) {
  float v = 0.f;
  if (i0 + e < a.V) {
    v = texp(__fsub_rn(bf16_bits_to_f32((d.lw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu), mx));
    if (MODE >= 1) {
      v = __fmul_rn(v, f);
      v = v < kFltMin ? 0.f : v;
      v = __fmul_rn(v, invZ);
    }
    if (MODE == 1) {
      v = __fsub_rn(v, d.qv[e]);
      v = v > 0.f ? v : 0.f;
    }
  }
  return v;
}
template <int MODE>
__device__ __forceinline__ float run_finish(const ResidualArgs& a, int ch, int lane, float mx, float f, float invZ, const RunData& d, float (&vals)[kRun]) {
  const int i0 = ch * kChunk + lane * kRun;
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < kRun; ++e) {
    vals[e] = r_value<MODE>(a, i0, mx, f, invZ, d, e);
    s = __fadd_rn(s, vals[e]);
  }
  return s;
}
// Elements [E0, E1) of the run's values into out[e * 64 + lane] (element-major: conflict-free).
template <int MODE, int E0, int E1>
__device__ __forceinline__ void run_part(const ResidualArgs& a, int row, int ch, int lane, float mx, float f, float invZ, float* out) {
  RunData d;
  run_load<MODE>(a, row, ch, lane, d);
  const int i0 = ch * kChunk + lane * kRun;
#pragma unroll
  for (int e = E0; e < E1; ++e) out[e * 64 + lane] = r_value<MODE>(a, i0, mx, f, invZ, d, e);
}
template <int MODE>
__device__ __forceinline__ float run_values(const ResidualArgs& a, int row, int ch, int lane, float mx, float f, float invZ, float (&vals)[kRun]) {
  RunData d;
  run_load<MODE>(a, row, ch, lane, d);
  return run_finish<MODE>(a, ch, lane, mx, f, invZ, d, vals);
}

// A group of 4 chunk values into one lane: lane l gets chunks 4 l .. 4 l + 3 of src (zeros past
// n; agent-scope loads at clamped addresses, all issued together).
__device__ __forceinline__ void gather_group(const float* src, int n, float (&g)[4]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = 4 * lane + k;
    const float v = ws_ld(src + (c < n ? c : n - 1));
    g[k] = c < n ? v : 0.f;
  }
}

// Sum of the 64 lanes' run sums in lane order (every lane gets it).
__device__ __forceinline__ float chunk_total(float run_sum) {
  const float r[1] = {run_sum};
  return wave_seq_sum(r);
}

// The row's chunk sums (n <= kMaxChunks) into registers of the wave: lane l gets chunks l,
// l + 64, ..., zeros past n (agent-scope loads: other workgroups wrote them).
__device__ __forceinline__ void gather_chunks(const float* src, int n, float (&r)[kMaxChunks / 64]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 0; k < kMaxChunks / 64; ++k) {
    const int c = 64 * k + lane;
    const float v = ws_ld(src + (c < n ? c : n - 1));  // unconditional (see merge_lists_top64)
    r[k] = c < n ? v : 0.f;
  }
}

// Phases 2 and 3 run one wave per 1024-element chunk, kWavesRes chunks to a workgroup (fewer
// arrivals at each counter: same-address atomics serialize), and the tails on wave 0.
constexpr int kWavesRes = 4;
__host__ __device__ constexpr int nq_res(int nch) { return (nch + kWavesRes - 1) / kWavesRes; }

// arrive_last for one wave (the other waves of the workgroup have left).
__device__ __forceinline__ bool arrive_last_wave(int* cnt, int total) {
  __builtin_amdgcn_s_waitcnt(0);
  int last = 0;
  if ((threadIdx.x & 63) == 0) {
    handoff_release();
    const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == total - 1;
    if (last) {
      __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      handoff_acquire();
    }
  }
  return __builtin_amdgcn_readfirstlane(last) != 0;
}

__global__ __launch_bounds__(64 * kWavesRes) void residual_phase2_kernel(ResidualArgs a) {
  const int nq = nq_res(a.nch);
  const int row = blockIdx.x / nq, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ch = (blockIdx.x % nq) * kWavesRes + wave;
  const int K = a.M - 1;
  const int64_t spec_l = lane < K ? a.spec[lane + 1] : -1;  // the finish's drafts, loaded up front
  if (ch < a.nch) {
    RunData d;
    run_load<0>(a, row, ch, lane, d);
    const int i0 = ch * kChunk + lane * kRun;
    const float mc = chunk_max(a, ch, lane, d);
    float vals[kRun];
    const float rs = run_finish<0>(a, ch, lane, mc, 1.f, 1.f, d, vals);
    const float ct = chunk_total(rs);
    if (row < K) {
      // the wave whose chunk holds draft d keeps a(d), q(d) and the chunk's maximum
      const int64_t dd = __shfl(spec_l, row);
      if (dd >= i0 && dd < i0 + kRun) {
        ws_st(a.a_draft + row, vals[dd - i0]);
        ws_st(a.q_draft + row, a.q[(size_t)row * a.V + dd]);
        ws_st(a.m_draft + row, mc);
      }
    }
    if (lane == 0) {
      ws_st(a.A + (size_t)row * a.nch + ch, ct);
      ws_st(a.mc + (size_t)row * a.nch + ch, mc);
    }
  }
  if (!arrive_last(a.cnt_rows + row * kCntStride, nq)) return;
  if (wave) return;
  // M, then Z over the groups of 4 chunks (lane l: group l): f_c A_c in chunk order within the
  // group, then the groups in order
  float Ag[4], Mg[4];
  gather_group(a.A + (size_t)row * a.nch, a.nch, Ag);
  gather_group(a.mc + (size_t)row * a.nch, a.nch, Mg);
  float m = -INFINITY;
#pragma unroll
  for (int k = 0; k < 4; ++k) m = 4 * lane + k < a.nch ? fmaxf(m, Mg[k]) : m;
  const float M = wave_max_f32(m);
  float G = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float S = 4 * lane + k < a.nch ? __fmul_rn(texp(__fsub_rn(Mg[k], M)), Ag[k]) : 0.f;
    G = k == 0 ? S : __fadd_rn(G, S);
  }
  const float g1[1] = {G};
  const float Zrow = wave_seq_sum(g1);
  if (lane == 0) {
    ws_st(a.Z + row, Zrow);
    ws_st(a.rowmax + row, M);
  }
}

// Phase 3: n from the accept tests, then one row j = n (the first rejected draft's row, or the
// bonus row K): chunk sums of r, then the last workgroup draws the token with u[K] by a blocked
// inverse-CDF search (group, chunk, run, element).
__global__ __launch_bounds__(64 * kWavesRes) void residual_phase3_kernel(ResidualArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int ch = blockIdx.x * kWavesRes + wave;
  const int K = a.M - 1;
  // The accept test, every draft at once, in every wave (one round trip for all its loads and
  // every row's max and Z): n = the drafts that pass before the first that fails, where an
  // out-of-vocabulary draft fails.
  const int rl = lane < a.M ? lane : 0, dl = lane < K ? lane : 0;
  const float mx_l = ws_ld(a.rowmax + rl), z_l = ws_ld(a.Z + rl);
  const float a_l = ws_ld(a.a_draft + dl), q_l = ws_ld(a.q_draft + dl), md_l = ws_ld(a.m_draft + dl);
  const float u_l = a.u[dl];
  const int64_t d_l = a.spec[dl + 1];
  const float uK = a.u[K];
  float e_d = __fmul_rn(a_l, texp(__fsub_rn(md_l, mx_l)));
  e_d = e_d < kFltMin ? 0.f : e_d;
  const float iz_l = __fdiv_rn(1.f, z_l);
  const bool pass = lane < K && d_l >= 0 && d_l < a.V && __fmul_rn(u_l, q_l) < __fmul_rn(e_d, iz_l);
  const int j = __builtin_ctzll(~__ballot(pass));  // <= K: lanes from K on do not pass
  const float Mj = lane_val(mx_l, j), izj = lane_val(iz_l, j);  // fl(1 / Z_j)
  const float* mcj = a.mc + (size_t)j * a.nch;
  float vals[kRun];
  if (ch < a.nch) {
    // the chunk maximum again from the loaded words (phase 2's value, without a workspace load)
    RunData d;
    if (j < K) run_load<1>(a, j, ch, lane, d);
    else run_load<2>(a, j, ch, lane, d);
    const float mc = chunk_max(a, ch, lane, d);
    const float f = texp(__fsub_rn(mc, Mj));
    const float rs = j < K ? run_finish<1>(a, ch, lane, mc, f, izj, d, vals) : run_finish<2>(a, ch, lane, mc, f, izj, d, vals);
    const float ct = chunk_total(rs);
    if (lane == 0) ws_st(a.chunk_sum + ch, ct);
  }
  if (!arrive_last(a.cnt_all, gridDim.x)) return;
  // The last workgroup: wave 0 runs the exact chain over the group sums while waves 1-3 compute
  // the values of the chunk that an unordered (parallel) scan finds, a third of each run each;
  // the exact search lands on that chunk in all but rounding ties (wave 0 then computes its own).
  __shared__ float sp_vals[kChunk];
  __shared__ int sp_chunk;
  __shared__ __align__(16) float chain_lds[64];
  float c4[4], pre1[1], G1[1];
  if (wave) {
    // lane l: group l (chunk sums and maxima); an inclusive shuffle scan over the groups, then
    // the chunk within the chosen group, both in any order
    float cw[4], mw[4];
    gather_group(a.chunk_sum, a.nch, cw);
    gather_group(mcj, a.nch, mw);
    const float gs = ((cw[0] + cw[1]) + cw[2]) + cw[3];
    float ps = gs;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float y = __shfl_up(ps, o);
      if (lane >= o) ps += y;
    }
    const float tgt = uK * lane_val(ps, 63);
    const unsigned long long over = __ballot(ps > tgt);
    const unsigned long long pos = __ballot(gs > 0.f);
    const int gg = over ? __ffsll((long long)over) - 1 : (pos ? 63 - __clzll((long long)pos) : 0);
    float acc = lane_val(ps, gg) - lane_val(gs, gg);
    int kk = 3;
#pragma unroll
    for (int k = 3; k >= 0; --k) {
      const float v = lane_val(cw[k], gg);
      kk = v > 0.f ? k : kk;  // fallback: the first positive chunk of the group
    }
    bool found = false;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float v = lane_val(cw[k], gg);
      if (!found && acc + v > tgt && v > 0.f) {
        kk = k;
        found = true;
      }
      acc += v;
    }
    const int cg = 4 * gg + kk;
    float mg = lane_val(mw[0], gg);
#pragma unroll
    for (int k = 1; k < 4; ++k) mg = kk == k ? lane_val(mw[k], gg) : mg;
    const float fg = texp(__fsub_rn(mg, Mj));
    if (j < K) {
      if (wave == 1) run_part<1, 0, 6>(a, j, cg, lane, mg, fg, izj, sp_vals);
      else if (wave == 2) run_part<1, 6, 11>(a, j, cg, lane, mg, fg, izj, sp_vals);
      else run_part<1, 11, 16>(a, j, cg, lane, mg, fg, izj, sp_vals);
    } else {
      if (wave == 1) run_part<2, 0, 6>(a, j, cg, lane, mg, fg, izj, sp_vals);
      else if (wave == 2) run_part<2, 6, 11>(a, j, cg, lane, mg, fg, izj, sp_vals);
      else run_part<2, 11, 16>(a, j, cg, lane, mg, fg, izj, sp_vals);
    }
    if (wave == 1 && lane == 0) sp_chunk = cg;
  } else {
    // lane l: group l's chunk sums, its sum in chunk order, then the exact chain over the groups
    gather_group(a.chunk_sum, a.nch, c4);
    float G = c4[0];
#pragma unroll
    for (int k = 1; k < 4; ++k) G = __fadd_rn(G, c4[k]);
    G1[0] = G;
    wave_seq_prefix(G1, 0.f, pre1, chain_lds);  // the running sums, the last the total
  }
  __syncthreads();
  if (wave) return;
  const float R = lane_val(pre1[0], 63);
  const bool degenerate = !(R > 0.f);
  const float target = __fmul_rn(uK, R);
  int pick = -1;
  if (!degenerate) {
    float acc;
    const int g = wave_seq_choose(G1, pre1, 0.f, target, &acc);  // the group
    // its chunk: the first whose running sum from acc exceeds the target, else the last positive
    float cg4[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) cg4[k] = lane_val(c4[k], g);
    int kc = -1;
    float a0 = acc;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (kc < 0) {
        const float t = __fadd_rn(a0, cg4[k]);
        if (t > target) kc = k;
        else a0 = t;
      }
    }
    if (kc < 0) {
      int last = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) last = cg4[k] > 0.f ? k : last;
      kc = last;
      a0 = acc;
#pragma unroll
      for (int k = 0; k < 4; ++k) a0 = k < kc ? __fadd_rn(a0, cg4[k]) : a0;
    }
    acc = a0;
    const int c = 4 * g + kc;
    float rs_l = 0.f;
    if (c == sp_chunk) {
#pragma unroll
      for (int e = 0; e < kRun; ++e) {
        vals[e] = sp_vals[e * 64 + lane];
        rs_l = __fadd_rn(rs_l, vals[e]);  // run_finish's sum
      }
    } else {
      const float mc = ws_ld(mcj + c), f = texp(__fsub_rn(mc, Mj));
      rs_l = j < K ? run_values<1>(a, j, c, lane, mc, f, izj, vals) : run_values<2>(a, j, c, lane, mc, f, izj, vals);
    }
    const float rr[1] = {rs_l};
    float run_acc;
    const int run = wave_seq_search(rr, acc, target, &run_acc, chain_lds);
    if (lane == run) {
      float x = run_acc;
      int last_nz = -1;
      for (int e = 0; e < kRun; ++e) {
        if (vals[e] > 0.f) last_nz = e;
        x = __fadd_rn(x, vals[e]);
        if (x > target) {
          pick = c * kChunk + lane * kRun + e;
          break;
        }
      }
      if (pick < 0) pick = c * kChunk + lane * kRun + last_nz;
    }
    pick = __builtin_amdgcn_readlane(pick, run & 63);  // run >= 0: chunk c's sum is positive
  } else {
    // degenerate residual (all zero): the row's argmax, first index on ties (keys are unique)
    const uint16_t* lg = a.logits + (size_t)j * a.V;
    uint64_t b = 0;
    for (int i = lane; i < a.V; i += 64) {
      const uint64_t k = vkey(ord16(lg[i]), i);
      b = k > b ? k : b;
    }
    pick = (int)vkey_idx(wave_max_u64(b));
  }
  {
    // lane i writes output i (a one-lane loop waited for each draft token load in turn)
    const int n = j;  // drafts a.spec[1..n] were accepted
    const int64_t base = *a.o.pos;
    if (lane < a.M) {
      a.o.tokens[lane] = lane < n ? a.spec[lane + 1] : (lane == n ? pick : -1);
      a.o.commit[lane] = lane <= n ? base + lane : -1;
    }
    if (lane == 0) {
      *a.o.n_accepted = n;
      *a.o.tok = pick;
      *a.o.pos = base + n + 1;
      *a.o.slot = n;
    }
  }
}

// ------------------------------------------------------------------ tree KV commit

// Moves the accepted path's rows to consecutive positions: for every plane (layer x kv head),
// row base + commit[t] -> row base + t for t = 1..n, where base = pos - n - 1 (pos already
// advanced by the accept kernel). Rows are read into registers before any is written.
// A commit that would touch rows outside the cache, or more than max_n rows, moves nothing and
// sets *status (when given) to 1; status is left alone otherwise.
__global__ void commit_rows_kernel(uint8_t* data, int planes, long plane_stride, int row_bytes, const int64_t* pos,
                                   const int64_t* n_accepted, const int64_t* commit, int max_n, int* status) {
  const int plane = blockIdx.x;
  if (plane >= planes) return;
  const int n = (int)*n_accepted;
  const int64_t base = *pos - n - 1;
  const int64_t max_len = plane_stride / row_bytes;
  bool bad = n > max_n || n < 0;
  for (int t = 1; t <= n && t <= max_n; ++t)
    bad |= base < 0 || base + commit[t] >= max_len || base + t >= max_len || commit[t] < 0;
  if (bad) {
    if (status && plane == 0 && threadIdx.x == 0) *status = 1;
    return;
  }
  uint8_t* p = data + (size_t)plane * plane_stride;
  // each thread moves 4-byte words; row_bytes % 4 == 0
  const int words = row_bytes / 4;
  for (int w0 = 0; w0 < words; w0 += blockDim.x) {
    const int w = w0 + threadIdx.x;
    uint32_t v[32];
    for (int t = 1; t <= n && t <= max_n; ++t)
      if (w < words) v[t - 1] = ((const uint32_t*)(p + (size_t)(base + commit[t]) * row_bytes))[w];
    __syncthreads();
    for (int t = 1; t <= n && t <= max_n; ++t)
      if (w < words) ((uint32_t*)(p + (size_t)(base + t) * row_bytes))[w] = v[t - 1];
    __syncthreads();
  }
}

}  // namespace tr

// ------------------------------------------------------------------ C ABI
using namespace tr;

namespace {

// Workspace layout (bytes): [0, kCntBytes) int32 counters (zero between calls), one per
// 256-byte line so that atomics on different counters never share a cache line (agent-scope
// atomics on one line serialize); then the largest of the per-kernel scratch areas.
constexpr size_t kCntBytes = 160 * kCntStride * sizeof(int);

int nch_top(int V) { return (V + kTopChunk - 1) / kTopChunk; }
int arg_chunk(int M) { return M <= 8 ? kArgChunkSmall : kArgChunkLarge; }
int nch_arg(int V, int M) { return (V + arg_chunk(M) - 1) / arg_chunk(M); }
int nch_run(int V) { return (V + kChunk - 1) / kChunk; }
// the argmax kernel's chunk keys [M * nch_arg] and row predictions [M]
size_t argmax_bytes(int M, int V) { return (size_t)M * nch_arg(V, M) * 8 + (size_t)M * 8; }

size_t scratch_bytes(int M, int V) {
  const size_t argmax = argmax_bytes(M, V) + (size_t)M * 4;
  const size_t samp = (size_t)M * nch_top(V) * kCand * 8 + (size_t)M * 8;
  const size_t resid = ((size_t)2 * M * nch_run(V) + nch_run(V) + (size_t)5 * M) * 4;
  size_t m = argmax > samp ? argmax : samp;
  m = m > resid ? m : resid;
  return (m + 255) & ~(size_t)255;
}

struct WsView {
  int* cnt;
  char* scratch;
};

bool ws_view(void* ws, size_t bytes, int M, int V, WsView* v) {
  if (!ws || bytes < kCntBytes + scratch_bytes(M, V)) return false;
  v->cnt = (int*)ws;  // counter c lives at cnt[c * kCntStride]
  v->scratch = (char*)ws + kCntBytes;
  return true;
}

// V <= 262144: at most 64 argmax chunk keys per row (one per lane of the reducing wave) and at
// most 64 top-64 lists per row
bool check_mv(int M, int V) { return M >= 1 && M <= 32 && V >= kCand && nch_arg(V, 1) <= 64 && nch_top(V) <= 64; }

AcceptOut make_out(int64_t* pred, int64_t* n, int64_t* tok, int64_t* pos, int64_t* slot, int64_t* tokens,
                   int64_t* commit) {
  AcceptOut o;
  o.pred = pred;
  o.n_accepted = n;
  o.tok = tok;
  o.pos = pos;
  o.slot = slot;
  o.tokens = tokens;
  o.commit = commit;
  return o;
}

// counters (in units of kCntStride ints): [0, 32) rows of the first kernel, [32] all-rows of
// the first kernel, [64, 96) rows of the residual phase 2, [128] phase 3.
int launch_argmax(const void* logits, int M, int V, int fin, const int64_t* spec, const int32_t* parent,
                  const WsView& w, const AcceptOut& o, hipStream_t st) {
  ArgmaxArgs a;
  a.logits = (const uint16_t*)logits;
  a.M = M;
  a.V = V;
  a.nch = nch_arg(V, M);
  a.fin = fin;
  a.spec = spec;
  a.parent = parent;
  a.keys = (uint64_t*)w.scratch;
  a.preds = (int64_t*)(w.scratch + (size_t)M * a.nch * 8);
  a.cnt_rows = w.cnt;
  a.cnt_all = w.cnt + 32 * kCntStride;
  a.o = o;
  if (arg_chunk(M) == kArgChunkSmall)
    hipLaunchKernelGGL(argmax_kernel<kArgChunkSmall>, dim3(M * a.nch), dim3(256), 0, st, a);
  else
    hipLaunchKernelGGL(argmax_kernel<kArgChunkLarge>, dim3(M * a.nch), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // namespace

extern "C" {

size_t tr_accept_workspace_bytes(int M, int V) {
  if (!check_mv(M, V)) return 0;
  return kCntBytes + scratch_bytes(M, V);
}

int tr_argmax_rows(const void* logits, int M, int V, void* ws, size_t ws_bytes, int64_t* pred, void* stream) {
  WsView w;
  if (!check_mv(M, V)) return TR_ERR_SHAPE;
  if (!logits || !pred || !ws_view(ws, ws_bytes, M, V, &w)) return TR_ERR_ARG;
  return launch_argmax(logits, M, V, FIN_NONE, nullptr, nullptr, w,
                       make_out(pred, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr), (hipStream_t)stream);
}

int tr_accept_greedy(const void* logits, int M, int V, const int64_t* spec_toks, void* ws, size_t ws_bytes,
                     int64_t* pred, int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot, int64_t* tokens,
                     int64_t* commit, void* stream) {
  WsView w;
  if (!check_mv(M, V)) return TR_ERR_SHAPE;
  if (!logits || !spec_toks || !n_accepted || !tok || !pos || !slot || !tokens || !commit ||
      !ws_view(ws, ws_bytes, M, V, &w))
    return TR_ERR_ARG;
  return launch_argmax(logits, M, V, FIN_CHAIN, spec_toks, nullptr, w,
                       make_out(pred, n_accepted, tok, pos, slot, tokens, commit), (hipStream_t)stream);
}

int tr_accept_tree(const void* logits, int M, int V, const int64_t* node_toks, const int32_t* parent, void* ws,
                   size_t ws_bytes, int64_t* pred, int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot,
                   int64_t* tokens, int64_t* commit, void* stream) {
  WsView w;
  if (!check_mv(M, V)) return TR_ERR_SHAPE;
  if (!logits || !node_toks || !parent || !n_accepted || !tok || !pos || !slot || !tokens || !commit ||
      !ws_view(ws, ws_bytes, M, V, &w))
    return TR_ERR_ARG;
  return launch_argmax(logits, M, V, FIN_TREE, node_toks, parent, w,
                       make_out(pred, n_accepted, tok, pos, slot, tokens, commit), (hipStream_t)stream);
}

static int launch_sample(const void* logits, int M, int V, int fin, const float* temperature, const float* top_p,
                         const int64_t* top_k, const float* u, const int64_t* spec, void* ws, size_t ws_bytes,
                         int64_t* out, const AcceptOut& o, hipStream_t st) {
  WsView w;
  if (!check_mv(M, V)) return TR_ERR_SHAPE;
  if (!logits || !temperature || !top_p || !top_k || !u || !ws_view(ws, ws_bytes, M, V, &w)) return TR_ERR_ARG;
  SampleArgs a;
  a.logits = (const uint16_t*)logits;
  a.M = M;
  a.V = V;
  a.nch = nch_top(V);
  a.fin = fin;
  a.temperature = temperature;
  a.top_p = top_p;
  a.top_k = top_k;
  a.u = u;
  a.spec = spec;
  a.cand = (uint32_t*)w.scratch;
  a.preds = (int64_t*)(w.scratch + (size_t)M * a.nch * kCand * 8);
  a.cnt_rows = w.cnt;
  a.cnt_all = w.cnt + 32 * kCntStride;
  a.out = out;
  a.o = o;
  hipLaunchKernelGGL(sample_kernel, dim3(M * a.nch), dim3(256), 0, st, a);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_sample(const void* logits, int M, int V, const float* temperature, const float* top_p, const int64_t* top_k,
              const float* u, void* ws, size_t ws_bytes, int64_t* out, void* stream) {
  if (!out) return TR_ERR_ARG;
  return launch_sample(logits, M, V, FIN_NONE, temperature, top_p, top_k, u, nullptr, ws, ws_bytes, out,
                       make_out(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr), (hipStream_t)stream);
}

int tr_accept_sample(const void* logits, int M, int V, const int64_t* spec_toks, const float* temperature,
                     const float* top_p, const int64_t* top_k, const float* u, void* ws, size_t ws_bytes,
                     int64_t* pred, int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot, int64_t* tokens,
                     int64_t* commit, void* stream) {
  if (!spec_toks || !n_accepted || !tok || !pos || !slot || !tokens || !commit) return TR_ERR_ARG;
  return launch_sample(logits, M, V, FIN_CHAIN, temperature, top_p, top_k, u, spec_toks, ws, ws_bytes, nullptr,
                       make_out(pred, n_accepted, tok, pos, slot, tokens, commit), (hipStream_t)stream);
}

int tr_accept_residual(const void* logits, int M, int V, const float* q, const int64_t* spec_toks, const float* u,
                       void* ws, size_t ws_bytes, int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot,
                       int64_t* tokens, int64_t* commit, void* stream) {
  WsView w;
  if (!check_mv(M, V) || M < 2) return TR_ERR_SHAPE;
  if (!logits || !q || !spec_toks || !u || !n_accepted || !tok || !pos || !slot || !tokens || !commit ||
      !ws_view(ws, ws_bytes, M, V, &w))
    return TR_ERR_ARG;
  hipStream_t st = (hipStream_t)stream;
  ResidualArgs a;
  a.logits = (const uint16_t*)logits;
  a.q = q;
  a.spec = spec_toks;
  a.u = u;
  a.M = M;
  a.V = V;
  a.nch = nch_run(V);
  // workspace: A and mc [M * nch] each, phase 3's chunk sums [nch], then rowmax, Z, a_draft,
  // q_draft, m_draft [M] each
  float* r = (float*)w.scratch;
  a.A = r;
  a.mc = a.A + (size_t)M * a.nch;
  a.chunk_sum = a.mc + (size_t)M * a.nch;
  a.rowmax = a.chunk_sum + a.nch;
  a.Z = a.rowmax + M;
  a.a_draft = a.Z + M;
  a.q_draft = a.a_draft + M;
  a.m_draft = a.q_draft + M;
  a.cnt_rows = w.cnt + 64 * kCntStride;
  a.cnt_all = nullptr;  // phase 2 has no all-rows handshake
  a.o = make_out(nullptr, n_accepted, tok, pos, slot, tokens, commit);
  hipLaunchKernelGGL(residual_phase2_kernel, dim3(M * nq_res(a.nch)), dim3(64 * kWavesRes), 0, st, a);
  if (hipGetLastError() != hipSuccess) return TR_ERR_LAUNCH;
  a.cnt_all = w.cnt + 128 * kCntStride;
  hipLaunchKernelGGL(residual_phase3_kernel, dim3(nq_res(a.nch)), dim3(64 * kWavesRes), 0, st, a);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_commit_rows(void* data, int planes, long plane_stride_bytes, int row_bytes, const int64_t* pos,
                   const int64_t* n_accepted, const int64_t* commit, int max_n, int* status, void* stream) {
  if (!data || !pos || !n_accepted || !commit) return TR_ERR_ARG;
  if (planes < 1 || row_bytes < 4 || row_bytes % 4 || max_n < 0 || max_n > 32) return TR_ERR_SHAPE;
  hipLaunchKernelGGL(commit_rows_kernel, dim3(planes), dim3(256), 0, (hipStream_t)stream, (uint8_t*)data, planes,
                     plane_stride_bytes, row_bytes, pos, n_accepted, commit, max_n, status);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"
