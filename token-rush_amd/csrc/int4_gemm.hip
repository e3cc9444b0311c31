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
//   * An MFMA chain against a ones operand gives X = sum(x) per row and group, and the group
//     result is  s * E + (mn - 128 s) * X  in fp32, applied once per group.
//
// Rows of x beyond M are padding lanes (they load row M-1 and are never stored), so every
// output row is computed by the same instructions for every M of one row-tile count: row i
// of an M = 1 call is bit-identical to row i of an M = 16 call (the property the reference's
// tests/test_marlin.py:42-52 checks for Marlin), and likewise within M = 17..32.
//
// Weight layout ("quad layout", made once at load time by tr_pack_int4): the K/128 groups of a
// 16-row strip are padded to a multiple of four (padding groups have zero codes, scale and min,
// so they contribute exactly 0) and stored as quads of four groups, 4352 bytes each
// (34 cache lines of 128 B, so no line is shared by two loads):
//   packed[N/16][Gp/4][4352]
//   bytes [1024 t, 1024 t + 1024): the codes of group 4 q + t. Lane l's 16 bytes at 16 l hold
//     row l % 16 of the group as four 32-bit words; word j covers k0 = 32 j + 8 (l/16) .. k0 + 7
//     (so MFMA j contracts k in [32 j, 32 j + 32) and the matching activations of one row are 64
//     contiguous bytes) with code k0 + 2p in nibble p and k0 + 2p + 1 in
//     nibble p + 4 (p = 0..3), so (w >> 4p) & 0x000F000F is the bf16 pair (k0 + 2p, k0 + 2p + 1)
//     once the exponent is set.
//   bytes [4096, 4352): row i's scale (low 16 bits) and min (high 16 bits) of group 4 q + t at
//     4096 + 16 i + 4 t, so one 16-byte load gives a lane its row's parameters for all four groups.
// A wave reads one strip's four groups with four 16-byte loads per lane plus one 16-byte load
// of parameters, all at one scalar offset.
//
// Work split ("activation-stationary"): a workgroup owns every grid_n-th strip and a K slot; each
// of its W waves owns one K block of GW groups (GW = 4 for M <= 16, 2 above), loads that
// block's activations into registers once, then streams the strips' tiles for its block.
// After every few strips the waves' partial tiles are summed through LDS in fixed wave order
// (deterministic). With S > 1 slots, slots write fp32 partials: either the caller's
// [S, M, N] buffer (the contract of the reference's partials(), tokenrush/quant.py:381-391,
// tokenrush/marlin.py:158-168) or a workspace the last-arriving slot reduces into bf16.
#include "accept_common.h"

#include <mutex>

namespace tr {

// In-kernel timeline (a build with -DTR_TIMELINE only, `make timeline`): wave w of workgroup b
// writes s_memrealtime (100 MHz) at mark i to tr_tl_buf[(b * 16 + w) * kTlMarks + i]. Marks: 0
// entry, 1 launch constants ready, 2 activations staged, 3 the first two strips issued, 4
// prologue end (group sums), 5 + r strip r's MACs done (r < 11), 16 a batch's reduction done,
// 20 exit of the strip loop, 21 the activation loads issued, 22 past the barrier that orders
// them before the strips. The normal build has none of it.
#ifdef TR_TIMELINE
constexpr int kTlMarks = 24, kTlBlocks = 2048;
__device__ unsigned long long tr_tl_buf[kTlBlocks * 16 * kTlMarks];
#define TLM(i)                                                                                       \
  do {                                                                                               \
    const unsigned long long t_ = __builtin_amdgcn_s_memrealtime();                                  \
    if ((threadIdx.x & 63) == 0 && blockIdx.x < kTlBlocks)                                           \
      tr_tl_buf[((size_t)blockIdx.x * 16 + (threadIdx.x >> 6)) * kTlMarks + (i)] = t_;               \
  } while (0)
#else
#define TLM(i) \
  do {         \
  } while (0)
#endif

constexpr int kGroup = 128;
constexpr int kQuad = 4;                          // groups per quad
constexpr int kCodeBytes = 1024;                  // one group's codes for 16 rows
constexpr int kSmOff = kQuad * kCodeBytes;        // parameters of the quad's groups
constexpr int kQuadBytes = kSmOff + 16 * kQuad * 4;  // 4352 = 34 x 128 B
constexpr int kWsCounterStride = 32;  // ints between workspace counters: one per 128-byte line
                                      // (agent-scope atomics on one line serialize)
constexpr int kTailE = 4;      // last-arriver slot sum: outputs per thread per pass
constexpr int kTailS = 2;      // and partial slots loaded per step
constexpr int kMaxWaves = 12;   // 768 threads: leaves ~170 VGPRs per lane (3 waves per SIMD)

// Groups of a K-long row after padding to whole quads.
__host__ __device__ __forceinline__ int padded_groups(int K) { return (K / kGroup + kQuad - 1) / kQuad * kQuad; }

enum { OUT_BF16 = 0, OUT_PARTIAL = 1, OUT_BF16_VIA_WS = 2 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// One wave's GW groups of one strip: this lane's 16 code bytes per group and its row's
// scale | min << 16 per group.
template <int GW>
struct Strip {
  uint4 w[GW];
  uint32_t sm[GW];
};

// Loads go through a buffer resource: the strip's byte offset is wave-uniform (an SGPR), the
// lane offsets are loop-invariant VGPRs and the per-group steps are immediates, so no vector
// instruction computes addresses. nt (non-temporal): the weights are streamed once. The
// parameters are loaded first: every group's fold needs them, so vmcnt then lets the first
// group start as soon as its own codes arrive.
template <int GW>
__device__ __forceinline__ void load_strip(Strip<GW>& t, __amdgpu_buffer_rsrc_t rsrc, int soff, int lane_off,
                                           int sm_voff) {
  if (GW == 4) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, sm_voff, soff, 2 /* nt */);
    t.sm[0] = v.x;
    t.sm[1] = v.y;
    t.sm[2 % GW] = v.z;
    t.sm[3 % GW] = v.w;
  } else {
    const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(rsrc, sm_voff, soff, 2 /* nt */);
    t.sm[0] = v.x;
    t.sm[1] = v.y;
  }
#pragma unroll
  for (int gw = 0; gw < GW; ++gw) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rsrc, lane_off + gw * kCodeBytes, soff, 2 /* nt */);
    t.w[gw] = make_uint4(v.x, v.y, v.z, v.w);
  }
}

// Scale of a (scale | min << 16) word, fp32.
template <bool F16S>
__device__ __forceinline__ float sm_scale(uint32_t sm) {
  return F16S ? f16_bits_to_f32(sm & 0xFFFFu) : __uint_as_float(sm << 16);
}
template <bool F16S>
__device__ __forceinline__ float sm_min(uint32_t sm) {
  return F16S ? f16_bits_to_f32(sm >> 16) : __uint_as_float(sm & 0xFFFF0000u);
}

// E = sum over the group of x * (128 + q), then acc += s * E. The group's other term,
// (mn - 128 s) * sum(x), is added once per strip by min_fold.
template <int MT, bool F16S>
__device__ __forceinline__ void tile_mac(const uint4& w, uint32_t sm, const uint4 (&xa)[MT][4], f32x4 (&acc)[MT],
                                         uint32_t kExp128) {
  const uint32_t kMask = 0x000F000Fu;
  const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
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
  const float sf = sm_scale<F16S>(sm);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4 E = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      E = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[mt][j]), b[j], E, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[mt][r] = fmaf(sf, E[r], acc[mt][r]);
  }
}

// acc[m][n] += sum over the wave's groups t of (mn - 128 s)[n, t] * X[m, t], X = sum of x over
// group t: one 16 x 16 x 4 fp32 MFMA per row tile with the group slot as k. A (Xa) holds
// X[m = lane % 16][t = lane / 16]; B is built here: lane l takes its row's parameters of group
// slot l / 16 (slots >= GW carry zero).
template <int MT, int GW, bool F16S>
__device__ __forceinline__ void min_fold(const uint32_t (&sm)[GW], const float (&Xa)[MT], int slot, f32x4 (&acc)[MT]) {
  uint32_t w;
  if (GW == 4) {
    const uint32_t a01 = (slot & 1) ? sm[1] : sm[0];
    const uint32_t a23 = (slot & 1) ? sm[3 % GW] : sm[2 % GW];
    w = (slot & 2) ? a23 : a01;
  } else {
    w = slot == 0 ? sm[0] : slot == 1 ? sm[1 % GW] : 0u;
  }
  const float c1 = fmaf(-128.f, sm_scale<F16S>(w), sm_min<F16S>(w));  // mn - 128 s: removes the code offset
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(Xa[mt], c1, acc[mt], 0, 0, 0);
}

// Output elements of a strip range are numbered e = (s * M + m) * P + j (strip s, row m, column j
// of P = 8 or 16 per strip row). Thread t takes e = t, t + T, ...: its column j = t % P is fixed,
// and (m, s) advance by a fixed step, so the index needs one division per kernel instead of
// several per element (a 32-bit division by a runtime value is ~40 VALU instructions).
struct StripWalk {
  int m, s;         // current element's row and strip index
  int dm, ds;       // step T / P as rows and strips
  int M;
  // magicM = ceil(2^32 / M) (M > 1): q / M = umulhi(q, magicM) exactly for the q < 2^16 used here
  __device__ __forceinline__ StripWalk(int t, int lgP, int T, int M_, uint32_t magicM) : M(M_) {
    const int q = t >> lgP, dq = T >> lgP;
    s = M_ == 1 ? q : (int)__umulhi((uint32_t)q, magicM);
    m = q - s * M_;
    ds = M_ == 1 ? dq : (int)__umulhi((uint32_t)dq, magicM);
    dm = dq - ds * M_;
  }
  __device__ __forceinline__ void next() {
    m += dm;
    s += ds;
    if (m >= M) {
      m -= M;
      ++s;
    }
  }
};

struct GemmArgs {
  const uint16_t* x;      // bf16 [M, K]
  const uint8_t* packed;  // strip layout
  void* out;              // bf16 [M, N] or fp32 [S, M, N]
  float* ws_part;         // fp32 [S, M, N] workspace (OUT_BF16_VIA_WS)
  int* ws_cnt;            // one counter per workgroup row range (<= N/16), zero between calls
  int M, N, K, S, R;      // R = strips per workgroup
  // Launch constants computed on the host, so that the kernel's prologue (run by every wave,
  // on the CU's shared scalar unit) needs no division: row workgroups gn = grid / S, workgroups
  // rbi < rfull take R strips and the rest R - 1, K blocks nb = Gp / GW, the quad-row stride and
  // the weight's size in bytes, and ceil(2^32 / S), ceil(2^32 / M) for exact small quotients.
  int gn, rfull, nb, quad_stride, wbytes;
  uint32_t magicS, magicM;
  int RB;                 // strips per LDS reduction batch
  int mode;
  int silu;               // 1: gate/up pair layout, out = silu(gate) * up, bf16 [M, N / 2]
  // Fused argmax (S == 1): per-row (value, first index) max of the bf16 outputs; the last
  // workgroup reduces the per-workgroup keys and finishes the greedy accept when spec != null.
  int argmax;
  uint64_t* am_keys;      // [M, grid] workspace
  int* am_cnt;            // arrival counter, zero between calls
  const int64_t* spec;    // [M] committed token + drafts, or null (argmax only)
  AcceptOut o;            // o.pred [M] always; the rest when spec != null
  int xstage_off;         // byte offset of the activation staging area in dynamic LDS (M <= 8, M > 16)
};

// q / d for q < 2^16 and 1 <= d < 2^15, magic = ceil(2^32 / d) (d == 1 has no 32-bit magic).
__device__ __forceinline__ int udiv_small(uint32_t q, int d, uint32_t magic) {
  return d == 1 ? (int)q : (int)__umulhi(q, magic);
}

// One accumulator tile element: (mt, lane, r) -> output row m = 16 mt + 4 (lane / 16) + r,
// column n = 16 strip + lane % 16.
template <int MT, int GW, bool F16S, bool XSTAGE>
__global__ __launch_bounds__(768) void int4_gemm_kernel(GemmArgs a) {
  // 16-byte aligned: the dynamic area follows the kernel's 776 bytes of static LDS, and the
  // ring's and staging area's 16-byte accesses stall when misaligned (SQ_LDS_UNALIGNED_STALL)
  extern __shared__ __attribute__((aligned(16))) float red[];  // [2][RB][W][MT][64][4]
  TLM(0);
  __shared__ uint64_t rowbest[32];  // fused argmax: best key per output row
  if (threadIdx.x < 32) rowbest[threadIdx.x] = 0;
  const int G = a.K / kGroup;
  const int W = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int rbi = udiv_small(blockIdx.x, a.S, a.magicS);
  const int slot = blockIdx.x - rbi * a.S;
  // Workgroup rbi of the grid_n row workgroups takes strips rbi, rbi + grid_n, ...: at any
  // moment all workgroups stream one contiguous band of the weight, which keeps their progress
  // even (contiguous per-workgroup ranges finish up to 3 us apart on the large shapes).
  const int gn = a.gn;
  const int r0 = 0;
  const int r1 = rbi < a.rfull ? a.R : a.R - 1;
  auto phys = [&](int r) { return rbi + r * gn; };

  const int nb = a.nb;                                 // K blocks (GW divides a quad)
  const int b0 = udiv_small(slot * nb, a.S, a.magicS);
  const int b1 = udiv_small((slot + 1) * nb, a.S, a.magicS);
  const int nw = b1 - b0;                              // active waves of this slot
  const bool active = wave < nw;
  const int gbase = (b0 + min(wave, nw - 1)) * GW;     // first group of this wave's block

  const uint32_t kExp128 = vgpr_const(0x43004300u);

  // Byte offset of this wave's groups in strip r. Strips past the range get an offset beyond
  // the buffer resource's size: the hardware returns zeros for those loads without touching
  // memory, so every loop path issues the same loads (no vmcnt drain) and none re-reads HBM.
  const int quad_stride = a.quad_stride;
  const int blk_off = gbase / kQuad * kQuadBytes + gbase % kQuad * kCodeBytes;
  const int oob = a.wbytes;
  auto strip_off = [&](int r) { return __builtin_amdgcn_readfirstlane(r < r1 ? phys(r) * quad_stride + blk_off : oob); };
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)a.packed, (short)0, oob, 0x00020000);
  TLM(1);
  const int lane_off = 16 * lane;
  // parameters of row lane % 16, groups gbase % 4 .. + GW - 1, relative to the strip offset
  const int sm_voff = kSmOff + 16 * (lane & 15) + 4 * (gbase % kQuad) - (gbase % kQuad) * kCodeBytes;

  // Activations of this wave's K block, in registers for the whole strip loop, in the MFMA
  // A-operand layout (lane l: row l % 16 of its row tile, k = 32 j + 8 (l / 16) .. + 7 of MFMA j).
  // Padding groups (g >= G) read group G - 1: finite values that meet zero scale and min.
  uint4 xa[GW][MT][4];
  constexpr int kXL = MT == 1 ? 8 : 16;  // staging loads per wave: one per row (GW = 4), or per row pair (GW = 2)
  uint4 xv[kXL];                         // staged rows, held in VGPRs until they are written to LDS
  if constexpr (XSTAGE) {
    // M <= 8: load the rows coalesced into VGPRs, write them to this wave's LDS staging area,
    // then read them back in the operand layout. In the operand layout itself consecutive lanes
    // would read different rows, each lane a separate cache access, which took 3-6 us for these
    // 8 KB per wave. Loading straight into LDS (buffer_load ... lds) lands no earlier and made the
    // M = 8 layer set 0.8 us slower than this register round trip. Load t brings row t of the wave's four
    // groups (lane l: group l / 16, 16-byte chunk (l % 16) ^ t), so a call issues M loads, one per
    // real row: every load instruction costs the CU's address unit the same 16 cycles whether
    // its lanes fetch or not. The staging area holds row r of group gw at (r GW + gw) 256 bytes,
    // chunk k of the row in 16-byte slot k ^ r, so the 16 rows read by one operand load fall in
    // different LDS banks.
    //
    // M = 17..32 (two row tiles, two groups per wave): load u brings rows 2u and 2u + 1 (lanes
    // 0-31 and 32-63; lane l: group (l / 16) % 2, chunk (l % 16) ^ (row % 16)), all 16 loads
    // issued before the strips, and the 16-row tiles are staged one after the other through the
    // same 8 KB per wave. That area lies inside the reduction ring, which is first written after
    // the prologue (an LDS barrier orders them). Rows >= M load from beyond the resource: zeros.
    static_assert((MT == 1 && GW == 4) || (MT == 2 && GW == 2), "activation staging: 1 x 4 or 2 x 2 tiles");
    const auto xrs = __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.M * a.K * 2, 0x00020000);
    const int lk = lane & 15;
    if constexpr (MT == 1) {
      const int g = min(gbase + (lane >> 4), G - 1);
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if (t >= a.M) break;
        const int off = (t * a.K + g * kGroup) * 2 + ((lk ^ t) & 15) * 16;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
        xv[t] = make_uint4(v.x, v.y, v.z, v.w);
      }
    } else {
      const int g = min(gbase + ((lane >> 4) & 1), G - 1);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int row = 2 * u + (lane >> 5);
        const int off = row < a.M ? (row * a.K + g * kGroup) * 2 + ((lk ^ row) & 15) * 16 : 0x7FFFFFF0;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(xrs, off, 0, 0);
        xv[u] = make_uint4(v.x, v.y, v.z, v.w);
      }
    }
  } else {
#pragma unroll
    for (int gw = 0; gw < GW; ++gw) {
      const int g = min(gbase + gw, G - 1);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int xr = min(16 * mt + (lane & 15), a.M - 1);
        const uint4* p = (const uint4*)(a.x + (size_t)xr * a.K + g * kGroup + 8 * (lane >> 4));
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[gw][mt][j] = p[4 * j];  // k = 32 j + 8 (lane / 16) .. + 7
      }
    }
  }
  // Two strips in flight, issued after the activation loads (vmcnt counts loads in issue order,
  // so waiting for the activations leaves the strips in flight). Waves without a K block issue
  // out-of-range loads: no memory access, the same count.
  Strip<GW> buf[2];
  // Staged kernels: every wave's activation requests enter the CU's in-order memory pipeline
  // before any wave's weight requests, so no wave waits for its activations behind the other
  // waves' strips.
  TLM(21);
  if constexpr (XSTAGE) __builtin_amdgcn_s_barrier();
  TLM(22);
  load_strip<GW>(buf[0], rsrc, active ? strip_off(r0) : oob, lane_off, sm_voff);
  load_strip<GW>(buf[1], rsrc, active ? strip_off(r0 + 1) : oob, lane_off, sm_voff);
  TLM(3);
  if constexpr (XSTAGE) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * (GW + 1)) : "memory");  // the staging loads have landed
    TLM(2);
    char* stage = (char*)red + a.xstage_off + wave * (GW * 256 * (MT == 1 ? 8 : 16));
    const int i = lane & 15;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if constexpr (MT == 1) {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if (t >= a.M) break;
          *(uint4*)(stage + t * 1024 + lane * 16) = xv[t];  // lane l: chunk l % 16 of group l / 16
        }
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) *(uint4*)(stage + u * 1024 + lane * 16) = xv[8 * mt + u];  // rows 2u, 2u + 1
      }
#pragma unroll
      for (int gw = 0; gw < GW; ++gw) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = 4 * j + (lane >> 4);
          const int rs = MT == 1 ? (i & 7) : i;  // staged row
          const uint4 v = *(const uint4*)(stage + (rs * GW + gw) * 256 + ((k ^ i) & 15) * 16);
          xa[gw][mt][j] = 16 * mt + i < a.M ? v : make_uint4(0u, 0u, 0u, 0u);
        }
      }
    }
    if constexpr (MT == 2) lds_barrier();  // every wave's staging reads before any ring write
  }

  // Xa[mt] = sum of x over group gbase + lane / 16 for row 16 mt + lane % 16 (the A operand of
  // min_fold), from MFMAs with x as B and a block selector as A: rows 4 t .. 4 t + 3 of A are
  // ones against group slot t, so output row i holds the sum for slot i / 4.
  float Xa[MT];
  {
    const int sel = (lane & 15) >> 2;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      // one accumulator per group slot (independent MFMA chains); a lane's element of D is
      // nonzero in exactly one of them, so their sum is exact
      f32x4 D[GW];
#pragma unroll
      for (int gw = 0; gw < GW; ++gw) {
        const uint32_t one = sel == gw ? 0x3F803F80u : 0u;
        const bf16x8 A = __builtin_bit_cast(bf16x8, make_uint4(one, one, one, one));
        D[gw] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          D[gw] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, xa[gw][mt][j]), D[gw], 0, 0, 0);
      }
      float xs = D[0][0];
#pragma unroll
      for (int gw = 1; gw < GW; ++gw) xs += D[gw][0];
      Xa[mt] = xs;
    }
  }
  TLM(4);
  const int slot16 = lane >> 4;
  const StripWalk walk16(threadIdx.x, 4, blockDim.x, a.M, a.magicM), walk8(threadIdx.x, 3, blockDim.x, a.M, a.magicM);

  // Partial tiles of RB consecutive strips are collected in LDS and reduced together (one
  // barrier per batch); batches alternate between two halves of the LDS ring, so the next
  // batch's writes never race the previous batch's reads.
  const int RB = a.RB;
  int sib = 0, half = 0;  // position in the current batch, ring half (wave-uniform)
  for (int rb = r0; rb < r1; rb += 2) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = rb + h;
      f32x4 acc[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (active && r < r1) {
#pragma unroll
        for (int gw = 0; gw < GW; ++gw) tile_mac<MT, F16S>(buf[h].w[gw], buf[h].sm[gw], xa[gw], acc, kExp128);
        min_fold<MT, GW, F16S>(buf[h].sm, Xa, slot16, acc);
      }
#ifdef TR_TIMELINE
      if (r < 11) {
        asm volatile("" ::"v"(acc[0][0]), "v"(acc[0][3]));  // the strip's MACs before the stamp
        TLM(5 + r);
      }
#endif
      // The refill is issued on every path (out-of-range offsets for inactive waves and past the
      // range: zeros, no memory access), so every path has the same loads in flight and the
      // compiler's wait before the next strip's compute covers that strip's loads only -- a
      // refill under a branch made it wait for the other buffer's loads as well.
      load_strip<GW>(buf[h], rsrc, active ? strip_off(r + 2) : oob, lane_off, sm_voff);
      if (r < r1) {
        float* ring = red + (size_t)half * RB * W * MT * 256;
        if (active) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            *(f32x4*)(ring + ((size_t)(sib * W + wave) * MT + mt) * 256 + lane * 4) = acc[mt];
        }
        if (sib == RB - 1 || r == r1 - 1) {
          __syncthreads();
          const int ns = sib + 1, r_first = r - sib;
          // Sum over the nw waves' partial tiles, in wave order, of output (m, n16) of strip r_first + sidx.
          auto wave_sum = [&](int sidx, int m, int n16) {
            const int mt = m >> 4, mm = m & 15;
            const float* src = ring + ((size_t)sidx * W * MT + mt) * 256 + (16 * (mm >> 2) + n16) * 4 + (mm & 3);
            float part[kMaxWaves];
#pragma unroll
            for (int w = 0; w < kMaxWaves; ++w) part[w] = w < nw ? src[(size_t)w * MT * 256] : 0.f;
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < kMaxWaves; ++w)
              if (w < nw) v += part[w];
            return v;
          };
          if (a.silu && a.mode == OUT_BF16) {
            // pair layout: rows 0..7 of a strip are gate rows, 8..15 the matching up rows
            const int F = a.N / 2, j = threadIdx.x & 7;
            for (StripWalk w = walk8; w.s < ns; w.next()) {
              const int sidx = w.s, m = w.m;
              const float g = bf16_bits_to_f32(f32_to_bf16_bits(wave_sum(sidx, m, j)));
              const float u = bf16_bits_to_f32(f32_to_bf16_bits(wave_sum(sidx, m, j + 8)));
              ((uint16_t*)a.out)[(size_t)m * F + 8 * phys(r_first + sidx) + j] = f32_to_bf16_bits(silu_mul_f32(g, u));
            }
          } else {
            const int n16 = threadIdx.x & 15;
            for (StripWalk w = walk16; w.s < ns; w.next()) {
              const int sidx = w.s, m = w.m;
              const float v = wave_sum(sidx, m, n16);
              const int n = 16 * phys(r_first + sidx) + n16;
              if (a.mode == OUT_BF16) {
                const uint32_t b = f32_to_bf16_bits(v);
                if (a.out) ((uint16_t*)a.out)[(size_t)m * a.N + n] = (uint16_t)b;
                if (a.argmax) __hip_atomic_fetch_max(&rowbest[m], vkey(ord16(b), n), __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_WORKGROUP);
              }
              else if (a.mode == OUT_PARTIAL)
                ((float*)a.out)[((size_t)slot * a.M + m) * a.N + n] = v;
              else  // agent-scope store: written through to the coherence point, no L2 flush needed
                __hip_atomic_store(a.ws_part + ((size_t)slot * a.M + m) * a.N + n, v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
          }
          sib = 0;
          half ^= 1;
          TLM(16);
        } else {
          ++sib;
        }
      }
    }
  }

  if (a.argmax) {
    // Publish this workgroup's row keys; the last workgroup reduces them (fixed order is not
    // needed: a max of unique keys) and finishes the accept.
    __syncthreads();
    if (threadIdx.x < a.M) ws_st(a.am_keys + (size_t)threadIdx.x * gridDim.x + blockIdx.x, rowbest[threadIdx.x]);
    if (!arrive_last(a.am_cnt, gridDim.x)) return;
    __shared__ int64_t pred[32], spec[32];
    const int nwv = blockDim.x >> 6;
    for (int m = threadIdx.x >> 6; m < a.M; m += nwv) {
      // up to 8 keys per lane loaded unconditionally (clamped index), so all are in flight at
      // once; a loop of loads under its bound check waited for each in turn
      uint64_t best = 0;
      const int grid = (int)gridDim.x;
      for (int g0 = 0; g0 < grid; g0 += 512) {
        uint64_t k[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const int g = g0 + lane + 64 * q;
          k[q] = ws_ld(a.am_keys + (size_t)m * grid + (g < grid ? g : grid - 1));  // lanes on consecutive keys
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) best = (g0 + lane + 64 * q < grid && k[q] > best) ? k[q] : best;
      }
      best = wave_max_u64(best);
      if (lane == 0) {
        pred[m] = vkey_idx(best);
        a.o.pred[m] = pred[m];
      }
    }
    if (a.spec && threadIdx.x < a.M) spec[threadIdx.x] = a.spec[threadIdx.x];
    __syncthreads();
    if (a.spec && threadIdx.x < 64) finish_chain(pred, spec, a.M, a.o);
    return;
  }
  TLM(20);
  if (a.mode != OUT_BF16_VIA_WS) return;
  // Last-arriving slot of this row range sums the S partials in slot order -> bf16. The
  // partials were stored at agent scope; waiting for those stores to complete before the
  // counter increment makes them visible to the last arriver's agent-scope loads, without
  // the L2 write-back a full __threadfence would cost on every workgroup.
  __shared__ int last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    handoff_release();
    last = __hip_atomic_fetch_add(a.ws_cnt + rbi * kWsCounterStride, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           a.S - 1;
    if (last) handoff_acquire();
  }
  __syncthreads();
  TLM(19);
  if (!last) return;
  // Each thread takes kTailE outputs per pass and loads their partials kTailS slots at a time,
  // all loads of a step issued together (outputs past the range load the last output's partials
  // and store nothing), then adds them in slot order. A loop of dependent loads here waited for
  // each partial in turn. (The pair layout's silu outputs take slot_sum_kernel instead.)
  const int nstr = r1 - r0;
  const int j = threadIdx.x & 15;
  const size_t slot_stride = (size_t)a.M * a.N;
  for (StripWalk w = walk16; w.s < nstr;) {
    int mi[kTailE], ni[kTailE];
    size_t off[kTailE];
    bool live[kTailE];
#pragma unroll
    for (int i = 0; i < kTailE; ++i) {
      live[i] = w.s < nstr;
      mi[i] = live[i] ? w.m : a.M - 1;
      ni[i] = 16 * phys(r0 + (live[i] ? w.s : nstr - 1)) + j;
      off[i] = (size_t)mi[i] * a.N + ni[i];
      w.next();
    }
    float v[kTailE];
#pragma unroll
    for (int i = 0; i < kTailE; ++i) v[i] = 0.f;
    for (int s0 = 0; s0 < a.S; s0 += kTailS) {
      float p[kTailS][kTailE];
#pragma unroll
      for (int q = 0; q < kTailS; ++q) {
        const float* base = a.ws_part + (size_t)min(s0 + q, a.S - 1) * slot_stride;
#pragma unroll
        for (int i = 0; i < kTailE; ++i) p[q][i] = __hip_atomic_load(base + off[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int q = 0; q < kTailS; ++q)
#pragma unroll
        for (int i = 0; i < kTailE; ++i)
          if (s0 + q < a.S) v[i] += p[q][i];
    }
#pragma unroll
    for (int i = 0; i < kTailE; ++i) {
      if (!live[i]) break;
      ((uint16_t*)a.out)[(size_t)mi[i] * a.N + ni[i]] = f32_to_bf16_bits(v[i]);
    }
  }
  TLM(23);
  if (threadIdx.x == 0)
    __hip_atomic_store(a.ws_cnt + rbi * kWsCounterStride, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The gate/up pair layout with more than one K slot: the slots' fp32 partials [S, M, N] summed in
// slot order, four outputs per thread; output (m, 8 s + j) is silu(bf16(g)) * bf16(u) with g, u
// the sums of columns 16 s + j and 16 s + 8 + j (the epilogue's arithmetic). A second launch
// instead of the GEMM's last-arriver sum: that tail loads two partials per output, and at M = 32
// gate_up took 37.2-37.6 us with it against 35.0 us for partials plus this kernel. Plain out mode
// keeps the in-kernel sum (qkv 12.8-13.1 us with it, 13.1-14.3 us with a second launch).
__global__ __launch_bounds__(256) void slot_sum_kernel(const float* __restrict__ part, int S, int M, int N,
                                                       uint16_t* __restrict__ out) {
  const size_t slot = (size_t)M * N;
  const int F = N / 2;
  const size_t quads = (size_t)M * F / 4;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < quads; i += (size_t)gridDim.x * blockDim.x) {
    const size_t m = 4 * i / F;
    const int c = (int)(4 * i % F), sb = c >> 3, j = c & 7;  // j = 0 or 4
    const size_t off = m * N + 16 * sb + j;
    float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
    for (int q = 0; q < S; ++q) {
      const float4 p = *(const float4*)(part + q * slot + off), r = *(const float4*)(part + q * slot + off + 8);
      g.x += p.x; g.y += p.y; g.z += p.z; g.w += p.w;
      u.x += r.x; u.y += r.y; u.z += r.z; u.w += r.w;
    }
    const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
    uint32_t b[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      b[e] = f32_to_bf16_bits(silu_mul_f32(bf16_bits_to_f32(f32_to_bf16_bits(gv[e])), bf16_bits_to_f32(f32_to_bf16_bits(uv[e]))));
    *(uint2*)(out + 4 * i) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
  }
}

// ----------------------------------------------------------------------------- layout kernels

// Engine packing (uint8 [N, K/2], element 2j in the low nibble of byte j; tokenrush/quant.py:9-10)
// plus scale/min [N, K/128] -> quad layout. One thread per output 32-bit word (1088 per quad);
// padding groups are written as zeros.
// Engine row of packed row i (0..15) of strip `strip`: identity, or for the gate/up pair layout
// (F = N / 2 > 0) gate row 8 strip + i for i < 8 and up row F + 8 strip + i - 8 otherwise.
__host__ __device__ __forceinline__ size_t src_row(size_t strip, int i, int F) {
  return F > 0 ? (i < 8 ? 8 * strip + i : (size_t)F + 8 * strip + (i - 8)) : 16 * strip + i;
}

__global__ void pack_kernel(const uint32_t* __restrict__ q, const uint16_t* __restrict__ scale,
                            const uint16_t* __restrict__ mn, uint32_t* __restrict__ packed, int N, int K, int F) {
  const int G = K / kGroup, nq = padded_groups(K) / kQuad;
  constexpr int kWords = kQuadBytes / 4;
  const size_t total = (size_t)N / 16 * nq * kWords;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int d = i % kWords;
    const size_t quad = i / kWords;
    const size_t strip = quad / nq;
    const int q0 = (int)(quad % nq) * kQuad;
    if (d >= kSmOff / 4) {
      const int e = d - kSmOff / 4, g = q0 + (e & 3);
      const size_t n = src_row(strip, e >> 2, F);
      packed[i] = g < G ? (uint32_t)scale[n * G + g] | ((uint32_t)mn[n * G + g] << 16) : 0u;
      continue;
    }
    const int g = q0 + d / 256, j = d & 3, lane = (d & 255) >> 2;
    if (g >= G) {
      packed[i] = 0u;
      continue;
    }
    const size_t n = src_row(strip, lane & 15, F);
    const int k0 = g * kGroup + 32 * j + 8 * (lane >> 4);
    const uint32_t u = q[(n * K + k0) / 8];  // bytes b0..b3 = codes k0..k0+7
    uint32_t w = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t b = (u >> (8 * p)) & 0xFF;
      w |= (b & 0xF) << (4 * p);
      w |= (b >> 4) << (16 + 4 * p);
    }
    packed[i] = w;
  }
}

// Quad layout -> engine packing and scale/min (the inverse of pack_kernel; padding is dropped).
__global__ void unpack_kernel(const uint32_t* __restrict__ packed, uint32_t* __restrict__ q,
                              uint16_t* __restrict__ scale, uint16_t* __restrict__ mn, int N, int K, int F) {
  const int G = K / kGroup, nq = padded_groups(K) / kQuad;
  constexpr int kWords = kQuadBytes / 4;
  const size_t total = (size_t)N / 16 * nq * kWords;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int d = i % kWords;
    const size_t quad = i / kWords;
    const size_t strip = quad / nq;
    const int q0 = (int)(quad % nq) * kQuad;
    const uint32_t w = packed[i];
    if (d >= kSmOff / 4) {
      const int e = d - kSmOff / 4, g = q0 + (e & 3);
      if (g >= G) continue;
      const size_t n = src_row(strip, e >> 2, F);
      scale[n * G + g] = (uint16_t)(w & 0xFFFF);
      mn[n * G + g] = (uint16_t)(w >> 16);
      continue;
    }
    const int g = q0 + d / 256, j = d & 3, lane = (d & 255) >> 2;
    if (g >= G) continue;
    const size_t n = src_row(strip, lane & 15, F);
    const int k0 = g * kGroup + 32 * j + 8 * (lane >> 4);
    uint32_t u = 0;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t lo = (w >> (4 * p)) & 0xF, hi = (w >> (16 + 4 * p)) & 0xF;
      u |= (lo | (hi << 4)) << (8 * p);
    }
    q[(n * K + k0) / 8] = u;
  }
}

// dequantize_int4 (tokenrush/quant.py:47-53): w = round(round(q * s) + m), two roundings, from the
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

constexpr int kCUs = 256;          // MI355X compute units

// Bytes of the quad layout of an N x K weight.
size_t packed_bytes(int N, int K) { return (size_t)N / 16 * (padded_groups(K) / kQuad) * kQuadBytes; }

// Shapes the kernels take: whole 16-row strips and 128-wide groups, and a packed weight that
// 32-bit buffer offsets address.
bool shape_ok(int N, int K) {
  return N > 0 && K > 0 && N % 16 == 0 && K % kGroup == 0 && packed_bytes(N, K) < ((size_t)1 << 31);
}
constexpr int kWavesPerCU = 12;    // occupancy of the GEMM kernel (about 150 VGPRs per lane)
constexpr size_t kLdsBudget = 64 * 1024;  // LDS of the reduction ring
constexpr size_t kLdsMax = 152 * 1024;    // dynamic LDS of one workgroup: gfx950's 160 KB less the kernel's static LDS

struct Plan {
  int GW, S, W, R, grid_n;
};

// ceil(2^32 / d) for 2 <= d < 2^15 (udiv_small's magic; d == 1 is handled there without one).
uint32_t magic_div(int d) { return d <= 1 ? 0u : (uint32_t)((((uint64_t)1 << 32) + d - 1) / d); }

int group_block(int M) { return M > 16 ? 2 : 4; }

// Tiling of an N x K weight for M rows. Depends on M only through the row-tile count
// (M <= 16 or not), so rows are bit-identical for every M within each range.
bool make_plan(int N, int K, int M, int S_req, int R_req, Plan* p);

// The partial-mode plan (the caller sums the slots, so more K slots cost only their writes, not
// a last-arriver slot sum): the slot count from the default's up to 6 with the least work on the
// busiest CU, rounds of workgroups x strips x waves, the smaller count on ties. The staged M <= 8
// kernel also counts its prologue (activation staging and group sums, ending ~4.7 us after launch
// against ~1.2 us per strip) as kRampStrips strips per workgroup, which favours fewer waves per
// workgroup. Measured at M = 8 (graph of launches, us): the 5120 x 6144 projection 7.31 at 1
// slot, 9.55 at 2, 6.54 at the chosen 3, 7.43 at 4; 5120 x 17408 12.35 at 3, 11.93 at 4, 11.67
// at the chosen 5, 13.96 at 6 (M = 1: 11.6, 11.7, 10.47, 12.3). At M = 16 (unstaged) 5120 x 17408
// ran 14.13 at 4 and 14.35 at 5 slots, and keeps 4.
constexpr long kRampStrips = 3;
bool make_partial_plan(int N, int K, int M, Plan* p) {
  Plan best;
  if (!make_plan(N, K, M, 0, 0, &best)) return false;
  long best_cost = -1;
  const int s_max = 6;
  for (int S = best.S; S <= s_max; ++S) {
    Plan q;
    if (!make_plan(N, K, M, S, 0, &q)) continue;
    const long grid = (long)q.grid_n * q.S;
    const long rounds = (grid + kCUs - 1) / kCUs;
    const long cost = rounds * (q.R + (M <= 8 ? kRampStrips : 0)) * q.W;
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = q;
    }
  }
  *p = best;
  return true;
}

bool make_plan(int N, int K, int M, int S_req, int R_req, Plan* p) {
  const int nstrips = N / 16;
  p->GW = group_block(M);
  const int nb = padded_groups(K) / p->GW;
  int S = S_req > 0 ? S_req : (nb + kMaxWaves - 1) / kMaxWaves;
  if (S < 1) S = 1;
  if (S > nb) return false;
  const int W = (nb + S - 1) / S;
  if (W > kMaxWaves) return false;
  int R = R_req;
  if (R <= 0) {
    int wg_per_cu = kWavesPerCU / W;
    if (wg_per_cu < 1) wg_per_cu = 1;
    const long slots = (long)kCUs * wg_per_cu;
    long grid_n = (slots + S - 1) / S;
    if (grid_n > nstrips) grid_n = nstrips;
    R = (int)((nstrips + grid_n - 1) / grid_n);
  }
  p->S = S;
  p->W = W;
  p->R = R;
  p->grid_n = (nstrips + R - 1) / R;
  return true;
}

template <int MT, int GW, bool F16S, bool XSTAGE>
hipError_t launch_t(GemmArgs a, const Plan& p, hipStream_t stream) {
  const dim3 grid(p.grid_n * p.S), block(64 * p.W);
  const size_t per_strip = (size_t)p.W * MT * 256 * sizeof(float);
  // Ring budget: the staged kernel keeps 64 KB (its staging takes the rest); the others share
  // the CU's LDS among the workgroups the plan puts on one CU, so larger batches never cost
  // occupancy.
  // The two-tile staging area shares the ring (it is dead before the first partial is written).
  constexpr bool kShared = XSTAGE && MT == 2;
  const int wg_per_cu = p.W >= kWavesPerCU ? 1 : kWavesPerCU / p.W;
  int rb = (int)(((XSTAGE && !kShared) ? kLdsBudget : kLdsMax / wg_per_cu) / (2 * per_strip));
  a.RB = rb < 1 ? 1 : (rb > 4 ? 4 : rb);
  const size_t ring = 2 * a.RB * per_strip;
  const size_t stage = XSTAGE ? (size_t)p.W * GW * 256 * (MT == 1 ? 8 : 16) : 0;
  a.xstage_off = kShared ? 0 : (int)ring;
  const size_t lds = kShared ? (ring > stage ? ring : stage) : ring + stage;
  {
    // staging + ring, or a ring over 64 KB, exceed the default 64 KB of dynamic LDS: raise this
    // kernel's limit once
    static bool raised = false;
    if (!raised) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&int4_gemm_kernel<MT, GW, F16S, XSTAGE>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLdsMax);
      if (e != hipSuccess) return e;
      raised = true;
    }
    if (lds > kLdsMax) return hipErrorInvalidValue;
  }
  hipLaunchKernelGGL((int4_gemm_kernel<MT, GW, F16S, XSTAGE>), grid, block, lds, stream, a);
  return hipGetLastError();
}

hipError_t launch(const GemmArgs& a, const Plan& p, int scale_dtype, hipStream_t stream) {  // NOLINT
  const bool f16 = scale_dtype == 1;
  if (a.M > 16) return f16 ? launch_t<2, 2, true, true>(a, p, stream) : launch_t<2, 2, false, true>(a, p, stream);
  if (a.M <= 8) return f16 ? launch_t<1, 4, true, true>(a, p, stream) : launch_t<1, 4, false, true>(a, p, stream);
  return f16 ? launch_t<1, 4, true, false>(a, p, stream) : launch_t<1, 4, false, false>(a, p, stream);
}

}  // namespace

extern "C" {

int tr_gemm_plan(int N, int K, int M, int* S, int* W, int* R) {
  if (!shape_ok(N, K) || M < 1 || M > 32 || !S || !W || !R) return TR_ERR_SHAPE;
  Plan p;
  if (!make_plan(N, K, M, 0, 0, &p)) return TR_ERR_CONFIG;
  *S = p.S;
  *W = p.W;
  *R = p.R;
  return TR_OK;
}

size_t tr_packed_bytes(int N, int K) { return shape_ok(N, K) ? packed_bytes(N, K) : 0; }

int tr_partial_slots(int N, int K, int M) {
  Plan p;
  if (!shape_ok(N, K) || M < 1 || M > 32 || !make_partial_plan(N, K, M, &p)) return -1;
  return p.S;
}

// Workspace of an out-mode call with S > 1: kWsCounters int32 counters at offset 0 -- a fixed
// region no call ever uses for partials, so one zero-filled buffer serves calls of every shape
// -- then the fp32 partials [S, M, N].
constexpr int kWsCounters = 4096;
static size_t ws_counter_bytes() { return (size_t)kWsCounters * kWsCounterStride * sizeof(int); }

size_t tr_gemm_workspace_bytes(int N, int K, int M) {
  Plan p;
  if (!shape_ok(N, K) || M < 1 || M > 32 || !make_plan(N, K, M, 0, 0, &p)) return 0;
  if (p.S == 1) return 0;
  return ws_counter_bytes() + (size_t)p.S * M * N * sizeof(float);
}

struct ArgmaxOut {
  const int64_t* spec;
  AcceptOut o;
};

static int gemm_impl(const void* x, const void* packed, void* out, void* partials, void* workspace,
                     size_t workspace_bytes, int M, int N, int K, int group, int scale_dtype, int n_slots, int R,
                     int silu, void* stream, const ArgmaxOut* am = nullptr) {
  if (group != kGroup) return TR_ERR_CONFIG;
  if (M < 0 || M > 32 || !shape_ok(N, K)) return TR_ERR_SHAPE;
  if (silu && partials) return TR_ERR_ARG;
  if (silu && N % 32) return TR_ERR_SHAPE;
  if (M == 0) return TR_OK;
  if (!x || !packed || (am ? partials != nullptr : (!out == !partials))) return TR_ERR_ARG;
  if (scale_dtype != 0 && scale_dtype != 1) return TR_ERR_ARG;
  Plan p;
  if (!make_plan(N, K, M, n_slots, R, &p)) return TR_ERR_CONFIG;
  if (partials && p.S != n_slots) return TR_ERR_CONFIG;
  GemmArgs a;
  a.x = (const uint16_t*)x;
  a.packed = (const uint8_t*)packed;
  a.M = M;
  a.N = N;
  a.K = K;
  a.S = p.S;
  a.R = p.R;
  a.gn = p.grid_n;
  a.rfull = N / 16 - (p.R - 1) * p.grid_n;
  a.nb = padded_groups(K) / p.GW;
  a.quad_stride = padded_groups(K) / kQuad * kQuadBytes;
  a.wbytes = (int)packed_bytes(N, K);
  a.magicS = magic_div(p.S);
  a.magicM = magic_div(M);
  a.ws_part = nullptr;
  a.ws_cnt = nullptr;
  a.silu = silu;
  a.argmax = 0;
  a.am_keys = nullptr;
  a.am_cnt = nullptr;
  a.spec = nullptr;
  a.o = AcceptOut{};
  if (am) {
    // fused argmax: one K slot (the per-row keys come from complete outputs), keys after the
    // counter line of the workspace
    if (p.S != 1 || partials || silu) return TR_ERR_CONFIG;
    const size_t need = kWsCounterStride * sizeof(int) + (size_t)p.grid_n * M * sizeof(uint64_t);
    if (!workspace || workspace_bytes < need || !am->o.pred) return TR_ERR_ARG;
    if (am->spec && (!am->o.n_accepted || !am->o.tok || !am->o.pos || !am->o.slot || !am->o.tokens || !am->o.commit))
      return TR_ERR_ARG;
    a.argmax = 1;
    a.am_cnt = (int*)workspace;
    a.am_keys = (uint64_t*)((char*)workspace + kWsCounterStride * sizeof(int));
    a.spec = am->spec;
    a.o = am->o;
  }
  if (partials) {
    a.mode = OUT_PARTIAL;
    a.out = partials;
  } else if (p.S == 1) {
    a.mode = OUT_BF16;
    a.out = out;
  } else {
    const size_t need = ws_counter_bytes() + (size_t)p.S * M * N * sizeof(float);
    if (!workspace || workspace_bytes < need) return TR_ERR_ARG;
    if (p.grid_n > kWsCounters) return TR_ERR_CONFIG;
    if (silu) {
      // the K slots' partials into the workspace, then their sum and silu in a second launch
      float* part = (float*)((char*)workspace + ws_counter_bytes());
      a.mode = OUT_PARTIAL;
      a.out = part;
      a.silu = 0;
      if (launch(a, p, scale_dtype, (hipStream_t)stream) != hipSuccess) return TR_ERR_LAUNCH;
      const size_t quads = (size_t)M * (N / 2) / 4;
      const int blocks = (int)((quads + 255) / 256 < 2048 ? (quads + 255) / 256 : 2048);
      hipLaunchKernelGGL(slot_sum_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, part, p.S, M, N,
                         (uint16_t*)out);
      return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
    }
    a.mode = OUT_BF16_VIA_WS;
    a.out = out;
    a.ws_cnt = (int*)workspace;
    a.ws_part = (float*)((char*)workspace + ws_counter_bytes());
  }
  return launch(a, p, scale_dtype, (hipStream_t)stream) == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

}  // extern "C"

// ----------------------------------------------------------------------------- no-allocation variant
//
// tr_int4_gemm_noalloc takes its workspace from `scratch`, a fixed device array of this library,
// instead of a caller's buffer: the counter region (zero between calls) then the fp32 partials of
// the K slots. Every GPU that runs the library holds its own copy until the process ends. In host
// code `scratch` names a host-side stand-in, never the device memory: the device address comes
// from hipGetSymbolAddress, once per device, and only that address reaches a kernel.
namespace {

constexpr size_t kScratchBytes = (size_t)16 << 20;
static_assert(kScratchBytes > (size_t)4096 * 32 * sizeof(int), "scratch holds the counter region and partials");
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];  // the device address of `scratch` on each device, once looked up

__global__ void zero_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// The current device's scratch address. The first call on a device looks it up and clears the
// counter region with a fill kernel on `stream` (a kernel, not a memset, so that a first call
// under graph capture records a node that is valid on every replay).
int device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return TR_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return TR_ERR_LAUNCH;
    const int words = (int)(ws_counter_bytes() / sizeof(uint32_t));
    hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, stream, (uint32_t*)p, words);
    if (hipGetLastError() != hipSuccess) return TR_ERR_LAUNCH;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return TR_OK;
}

}  // namespace

extern "C" {

int tr_int4_gemm_noalloc(const void* x, const void* packed, void* out, int M, int N, int K, int group, int scale_dtype,
                         void* stream) {
  if (group != kGroup) return TR_ERR_CONFIG;
  if (M < 0 || M > 32 || !shape_ok(N, K)) return TR_ERR_SHAPE;
  if (M == 0) return TR_OK;
  const size_t need = tr_gemm_workspace_bytes(N, K, M);
  if (need > kScratchBytes) return TR_ERR_SCRATCH;
  void* ws = nullptr;
  if (need > 0) {
    const int rc = device_scratch((hipStream_t)stream, &ws);
    if (rc != TR_OK) return rc;
  }
  return gemm_impl(x, packed, out, nullptr, ws, need > 0 ? kScratchBytes : 0, M, N, K, group, scale_dtype, 0, 0, 0,
                   stream);
}

int tr_int4_gemm_ex(const void* x, const void* packed, void* out, void* partials, void* workspace,
                    size_t workspace_bytes, int M, int N, int K, int group, int scale_dtype, int n_slots, int R,
                    void* stream) {
  return gemm_impl(x, packed, out, partials, workspace, workspace_bytes, M, N, K, group, scale_dtype, n_slots, R, 0,
                   stream);
}

int tr_int4_gemm_silu(const void* x, const void* packed, void* out, void* workspace, size_t workspace_bytes, int M,
                      int N, int K, int group, int scale_dtype, void* stream) {
  return gemm_impl(x, packed, out, nullptr, workspace, workspace_bytes, M, N, K, group, scale_dtype, 0, 0, 1, stream);
}

size_t tr_lm_head_workspace_bytes(int N, int K, int M) {
  Plan p;
  if (!shape_ok(N, K) || M < 1 || M > 32 || !make_plan(N, K, M, 0, 0, &p) || p.S != 1) return 0;
  return kWsCounterStride * sizeof(int) + (size_t)p.grid_n * M * sizeof(uint64_t);
}

int tr_lm_head_greedy(const void* x, const void* packed, void* logits, void* workspace, size_t workspace_bytes,
                      int M, int N, int K, int group, int scale_dtype, const int64_t* spec_toks, int64_t* pred,
                      int64_t* n_accepted, int64_t* tok, int64_t* pos, int64_t* slot, int64_t* tokens,
                      int64_t* commit, void* stream) {
  if (M < 1) return TR_ERR_SHAPE;
  ArgmaxOut am{spec_toks, AcceptOut{pred, n_accepted, tok, pos, slot, tokens, commit}};
  return gemm_impl(x, packed, logits, nullptr, workspace, workspace_bytes, M, N, K, group, scale_dtype, 0, 0, 0, stream,
                   &am);
}

int tr_int4_gemm(const void* x, const void* packed, void* out, void* partials, void* workspace,
                 size_t workspace_bytes, int M, int N, int K, int group, int scale_dtype, int n_slots,
                 void* stream) {
  return tr_int4_gemm_ex(x, packed, out, partials, workspace, workspace_bytes, M, N, K, group, scale_dtype,
                         partials ? n_slots : 0, 0, stream);
}

static int grid_for(size_t work) {
  size_t b = (work + 255) / 256;
  if (b > 65536) b = 65536;
  if (b < 1) b = 1;
  return (int)b;
}

static int pack_impl(const void* qweight, const void* scale, const void* mn, void* packed, int N, int K, int F,
                     void* stream) {
  if (!qweight || !scale || !mn || !packed) return TR_ERR_ARG;
  if (!shape_ok(N, K) || (F && N % 32)) return TR_ERR_SHAPE;
  const size_t total = packed_bytes(N, K) / 4;
  hipLaunchKernelGGL(pack_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream, (const uint32_t*)qweight,
                     (const uint16_t*)scale, (const uint16_t*)mn, (uint32_t*)packed, N, K, F);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

static int unpack_impl(const void* packed, void* qweight, void* scale, void* mn, int N, int K, int F, void* stream) {
  if (!qweight || !packed || !scale || !mn) return TR_ERR_ARG;
  if (!shape_ok(N, K) || (F && N % 32)) return TR_ERR_SHAPE;
  const size_t total = packed_bytes(N, K) / 4;
  hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(total)), dim3(256), 0, (hipStream_t)stream,
                     (const uint32_t*)packed, (uint32_t*)qweight, (uint16_t*)scale, (uint16_t*)mn, N, K, F);
  return hipGetLastError() == hipSuccess ? TR_OK : TR_ERR_LAUNCH;
}

int tr_pack_int4(const void* qweight, const void* scale, const void* mn, void* packed, int N, int K, void* stream) {
  return pack_impl(qweight, scale, mn, packed, N, K, 0, stream);
}

int tr_unpack_int4(const void* packed, void* qweight, void* scale, void* mn, int N, int K, void* stream) {
  return unpack_impl(packed, qweight, scale, mn, N, K, 0, stream);
}

int tr_pack_int4_pairs(const void* qweight, const void* scale, const void* mn, void* packed, int N, int K,
                       void* stream) {
  return pack_impl(qweight, scale, mn, packed, N, K, N / 2, stream);
}

int tr_unpack_int4_pairs(const void* packed, void* qweight, void* scale, void* mn, int N, int K, void* stream) {
  return unpack_impl(packed, qweight, scale, mn, N, K, N / 2, stream);
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

#ifdef TR_TIMELINE
// The timeline buffer of a -DTR_TIMELINE build (device address, size in bytes).
void* tr_gemm_timeline(size_t* bytes) {
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(tr_tl_buf)) != hipSuccess) return nullptr;
  if (bytes) *bytes = sizeof(tr_tl_buf);
  return p;
}
#endif

}  // extern "C"
