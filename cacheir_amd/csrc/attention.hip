// Paged decode / prefill attention for gfx950.
//
// A query row is one token (batch * q_len rows).  One workgroup handles one
// (row, KV head, context split); all GQA query heads of the KV head are computed
// together, so each K/V page is read from HBM once.  The host picks the number of
// splits S: 1 whenever rows * kv_heads already fills the GPU (then the workgroup
// writes the final output and nothing goes through global memory), otherwise a
// few splits whose (max, sum, O) partials a small merge kernel combines.
//
// fp16 pools, head_dim 128 (Llama-3 / Qwen2 shapes), 8 wavefronts per workgroup:
//   * the split's context is cut into 32-token blocks dealt round-robin to the
//     wavefronts; a wavefront issues every K and V load of its block up front
//     (8 KiB of K and 8 KiB of V in flight, no branches: tiles past the end are
//     clamped to a valid page and masked);
//   * S = Q K^T on MFMA 16x16x32 f16: A = the group's query heads padded to 16
//     rows, B = a 16-token tile of K read straight from its page (token rows of
//     256 B); fp32 accumulate;
//   * softmax in base 2 (scale*log2(e) folded into the scores): exact within the
//     block, online (running max / rescale) across a wavefront's blocks; the row
//     max over a tile's 16 token lanes is a DPP reduction (no LDS round trips) and
//     the rescale factors are read out of their lane as scalars;
//   * O = P V on VALU: a lane owns 8 contiguous head dims of 4 token rows of each
//     tile (1 KiB contiguous per load instruction); P comes from the score lanes by
//     ds_bpermute shuffles, in fp16 with two heads per dword (l sums the same
//     rounded values); the four token groups are summed once at the end;
//   * the 8 wavefronts merge (max, sum, O) through LDS with log-sum-exp weights.
// Prefill (q_len > 1) on fp16 pools runs attn_prefill_f16_d128 instead: 128 query
// vectors of a sequence per workgroup over its blocks, both products on MFMA.
// fp32 pools and other head sizes (tiny-model parity path) use a plain VALU kernel
// over 128-token chunks that always writes partials, merged by the same kernel.
//
// Reference semantics: cacheir/backends/triton_kernels.py:174-217 (paged gather
// pool[page_table[b, t // P], kvh, t % P], GQA kvh = h // (Hq/Hkv), positions
// t < seq_len) and cacheir/runtime/cpu.py:342-377 (softmax(q.k * scale) v,
// prefill causal mask).
#include "common.hpp"

#include <math.h>

#include <atomic>
#include <mutex>

namespace cir {
namespace {

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// Max over the 16 lanes of each DPP row (lanes 16r .. 16r+15): swap neighbours, swap
// pairs, mirror the half rows, mirror the rows; every lane ends with its row's max.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));   // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_mov<0x4E>(v));   // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_mov<0x141>(v));  // row_half_mirror
  v = fmaxf(v, dpp_mov<0x140>(v));  // row_mirror
  return v;
}
// The same pattern as a sum: lane 16r of each row ends with the row's total (the
// other lanes too, summed in another order).
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_mov<0xB1>(v);
  v += dpp_mov<0x4E>(v);
  v += dpp_mov<0x141>(v);
  v += dpp_mov<0x140>(v);
  return v;
}
// Sums over the four rows of four values at once, by gfx950's lane-swap instructions
// (no LDS): v_permlane16_swap(a, b) leaves rows (a0, b0, a2, b2) and (a1, b1, a3, b3),
// v_permlane32_swap(x, y) leaves (x0, x1, y0, y1) and (x2, x3, y2, y3).  Row k of the
// result holds the total of v[k], summed (r0 + r1) + (r2 + r3) in every lane.
__device__ __forceinline__ float swap_sum16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                  false, false);
  const uint32_t r0 = r[0], r1 = r[1];  // (bit_cast of a vector element lvalue reads element 0)
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ float rows_sum4(const float (&v)[4]) {
  const float ab = swap_sum16(v[0], v[1]), cd = swap_sum16(v[2], v[3]);
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, ab), __builtin_bit_cast(uint32_t, cd),
                                                  false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

// 8 wavefronts of 32-token steps measured best on MI355X at config 4 (batch 32,
// 2048 tokens), against 64-token steps, 16 wavefronts of 16 tokens and a
// double-buffered pipeline.  A long streaming read peaks at ~7.0 TB/s on this part;
// a loads-only copy of this kernel's access pattern (same grid, pages and per-lane
// addresses) takes 47.4 us at config 4 (5.7 TB/s), and the kernel 50.0 us.
constexpr int kTiles = 2;             // 16-token MFMA tiles per wavefront step
constexpr int kBlock = 16 * kTiles;   // tokens per wavefront step
constexpr int kWaves = 8;             // wavefronts per workgroup (fp16 path)
constexpr int kChunk = 128;  // tokens per partial in the generic path
// Page-table entries a workgroup keeps in LDS (2 KiB at 8 wavefronts): one per thread, since every thread fills
// one entry (a split whose pages exceed the thread count reads the table directly); the row sort of the
// longest-first dispatch also ranks one row per thread in this array.
constexpr int kPtCache = 64 * kWaves;
constexpr int kMinSplitTokens = 256;
constexpr float kLog2e = 1.4426950408889634f;

// Tokens visible to query row `row`, clamped to what the page table can address.
__device__ __forceinline__ int visible_len(const int32_t* lens, int row, int q_len, int max_ctx) {
  const int b = row / q_len;
  const int s = row - b * q_len;
  return min(lens[b] - q_len + s + 1, max_ctx);
}

// ----------------------------------------------------------------------------
// fp16 pools, head_dim 128.  G = query heads per KV head (1..8).
// Fused decode input (optional): the QKV projection's fp32 split-k partials
// [splits][batch][(Hq + 2 Hkv) D] instead of a finished q.  The workgroup then sums
// its heads' partials, applies RoPE to q and k, appends the new k and v to their page
// and keeps q in LDS -- the work of the QKV epilogue kernel, in the same order and
// precision, for one (row, KV head) at a time.
struct QkvIn {
  const float* part;        // null: q is read from `q`
  int splits;
  const float* inv_freq;    // [D/2]
  const int32_t* positions; // [batch]: position of the new token
};

// Splits of the QKV partials a fused workgroup loads before its first K/V block;
// more splits are loaded when summed.
constexpr int kSumUnroll = 8;

// FUSED: q comes from the QKV partials in `qkv` (decode, q_len 1), else from `q`.
template <int G, bool FUSED>
__global__ __launch_bounds__(64 * kWaves) void attn_f16_d128(
    const f16* __restrict__ q, f16* __restrict__ kp, f16* __restrict__ vp,
    const int32_t* __restrict__ pt, const int32_t* __restrict__ lens, f16* __restrict__ out,
    float* __restrict__ part_o, float* __restrict__ part_ml, int q_len, int Hq, int Hkv, int P, int max_pages,
    int S, float scale_log2, int sort_rows, QkvIn qkv) {
  constexpr int D = 128;
  __shared__ float sm_m[kWaves][16];
  __shared__ float sm_l[kWaves][16];
  __shared__ float sm_o[kWaves][G][D];
  __shared__ __align__(16) f16 sm_q[G][D];
  __shared__ __align__(16) f16 sm_kn[D];  // fused: the new token's k and v
  __shared__ __align__(16) f16 sm_vn[D];
  __shared__ int sm_pt[kPtCache];

  const int split = blockIdx.x, kvh = blockIdx.y;
  // Rows in decreasing order of context (sort_rows: decode, rows <= one per thread, more
  // workgroups than CUs): workgroups are dispatched in blockIdx order as CUs free up,
  // so the longest rows start first and the short ones fill in behind them (longest
  // processing time first) instead of a long row starting last and running alone.
  // Row t's rank counts the rows longer than it, ties broken by index.
  int row = blockIdx.z;
  if (sort_rows) {
    const int n = gridDim.z, t = threadIdx.x;
    const int lt = t < n ? lens[t] : 0;
    sm_pt[t] = lt;  // (the page-table cache is filled later)
    __syncthreads();
    if (t < n) {
      int rank = 0;
      for (int j = 0; j < n; ++j) {
        const int lj = sm_pt[j];
        rank += (lj > lt || (lj == lt && j < t)) ? 1 : 0;
      }
      if (rank == (int)blockIdx.z) sm_m[0][0] = __builtin_bit_cast(float, t);
    }
    __syncthreads();
    row = __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sm_m[0][0]));
    __syncthreads();  // sm_pt and sm_m are written again below
  }
  // readfirstlane: the wavefront index is uniform, so block indices and page-table
  // lookups stay scalar (s_load, their own counter) instead of vector loads that
  // would retire in order behind the K/V loads in flight.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int li = lane & 15;  // score column (token in tile) / Q row (head in group)
  const int lg = lane >> 4;  // k-group of the MFMA operands; token group for P V
  const int L = visible_len(lens, row, q_len, max_pages * P);
  const int nblk = L > 0 ? (L + kBlock - 1) / kBlock : 0;
  const int per = (nblk + S - 1) / S;
  const int b0 = split * per, b1 = min(nblk, b0 + per);
  const int b = row / q_len;
  const int32_t* ptrow = pt + (size_t)b * max_pages;

  // One block of K/V operands (kTiles 16-token tiles) for one wavefront.
  struct Blk {
    f16x8 k[kTiles][4], v[kTiles][4];
  };
  // Issue every K load, then every V load, of block `blk` (K first: the scores need
  // only K, so they start while V is still arriving).  Tiles past the end re-read
  // the block's first tile (masked in the scores).
  // This split's page-table entries, cached in LDS when they fit (filled before the
  // first workgroup barrier; until then lookups read the table directly).
  const int pg0 = (b0 * kBlock) / P;
  const int pg1 = min(max_pages, (b1 * kBlock + P - 1) / P);
  const bool pt_cached = pg1 - pg0 <= kPtCache;
  bool pt_ready = false;
  auto page_of = [&](int t) __attribute__((always_inline)) {
    const int pi = t / P;
    return (pt_ready && pt_cached) ? __builtin_amdgcn_readfirstlane(sm_pt[pi - pg0]) : ptrow[pi];
  };
  auto page_bases = [&](size_t (&base)[kTiles], int blk) __attribute__((always_inline)) {
    const int tb = blk * kBlock;
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const int tj = tb + 16 * j;
      const int tv = tj < L ? tj : tb;
      const int page = page_of(tv);
      base[j] = (((size_t)page * Hkv + kvh) * P + (tv % P)) * D;
    }
  };
  auto load_k = [&](Blk& o, int blk) __attribute__((always_inline)) {
    size_t base[kTiles];
    page_bases(base, blk);
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const f16* krow = kp + base[j] + (size_t)li * D + 8 * lg;
#pragma unroll
      for (int s = 0; s < 4; ++s) o.k[j][s] = *reinterpret_cast<const f16x8*>(krow + 32 * s);
    }
  };
  auto load_v = [&](Blk& o, int blk) __attribute__((always_inline)) {
    size_t base[kTiles];
    page_bases(base, blk);
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const f16* vrow = vp + base[j] + 8 * li;
#pragma unroll
      for (int u = 0; u < 4; ++u) o.v[j][u] = *reinterpret_cast<const f16x8*>(vrow + (size_t)(4 * u + lg) * D);
    }
  };
  auto load_block = [&](Blk& o, int blk) __attribute__((always_inline)) {
    load_k(o, blk);
    load_v(o, blk);
  };
  // Issue order: load counters retire in order, so waiting for one load waits for every
  // load issued before it.  q (or the fused prologue's partials) and the page-table
  // entries for the LDS cache go out first, the first K/V block after them, and in a
  // workgroup with blocks every thread issues the same loads (indices clamped, results
  // unused where out of range), so the compiler's waits before the LDS fill and the
  // prologue's arithmetic count the block's loads out instead of waiting for them.
  //
  // Q as the MFMA A operand: row li = head kvh*G + li (zero rows past G); element e
  // of step s is head dim 32*s + 8*lg + e, the same mapping the K loads use.
  f16x8 qa[4];
  if constexpr (!FUSED) {
    const f16* qrow = q + ((size_t)row * Hq + (size_t)kvh * G + (li < G ? li : 0)) * D + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(qrow + 32 * s);
      qa[s] = (li < G) ? v : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  // Fused decode input: q, k, v of this row and KV head.  Work items are column pairs:
  // RoPE pair i of q head hh (hh < G) or of k (hh == G), then pairs of v (hh == G + 1).
  // The split whose blocks hold the new token (the writer) also computes its k and v:
  // they go to LDS, the wavefront whose block holds the token patches them into its
  // registers, and the writer appends them to the pool at the very end (a store
  // completes after loads issued later and would hold up every wait behind it), so
  // no ordering between the append and any load of that page line is needed.  The
  // first kSumUnroll splits of an item are loaded up front; more when it is summed.
  constexpr int kHalf = D / 2;
  constexpr int kItems = ((G + 2) * kHalf + 64 * kWaves - 1) / (64 * kWaves);  // per thread
  const int pos = FUSED ? qkv.positions[b] : 0;
  const bool writer = FUSED && split == min(S - 1, (pos / kBlock) / max(per, 1));
  const int items = writer ? (G + 2) * kHalf : G * kHalf;
  const int N = (Hq + 2 * Hkv) * D;
  const size_t plane = (size_t)gridDim.z * N;
  const float* prow = FUSED ? qkv.part + (size_t)row * N : nullptr;
  auto item_col = [&](int it) __attribute__((always_inline)) -> size_t {  // first column of item it
    const int hh = it / kHalf, i = it - hh * kHalf;
    return (hh < G ? ((size_t)kvh * G + hh) * D : (size_t)(Hq + (hh - G) * Hkv) * D + (size_t)kvh * D) + 2 * i;
  };
  float xa[kItems][kSumUnroll], xb[kItems][kSumUnroll], fr[kItems];
  if constexpr (FUSED) {
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int it = min((int)threadIdx.x + k * 64 * kWaves, items - 1);
      const float* p = prow + item_col(it);
#pragma unroll
      for (int s = 0; s < kSumUnroll; ++s) {
        const float* ps = p + (size_t)(s < qkv.splits ? s : 0) * plane;
        xa[k][s] = ps[0];
        xb[k][s] = ps[1];
      }
      fr[k] = qkv.inv_freq[it % kHalf];
    }
  }
  // Sums each item's partials in split order (bitwise as the QKV epilogue kernel),
  // applies RoPE and puts q (and the writer's k and v) in LDS.
  auto prologue = [&]() __attribute__((always_inline)) {
    auto sum = [&](const float (&t)[kSumUnroll], size_t col) __attribute__((always_inline)) {
      float v = t[0];
#pragma unroll
      for (int s = 1; s < kSumUnroll; ++s)
        if (s < qkv.splits) v += t[s];
      for (int s = kSumUnroll; s < qkv.splits; ++s) v += prow[(size_t)s * plane + col];
      return v;
    };
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
      const int it = threadIdx.x + k * 64 * kWaves;
      if (it >= items) continue;
      const int hh = it / kHalf, i = it - hh * kHalf;
      const size_t col = item_col(it);
      const float x0 = sum(xa[k], col), x1 = sum(xb[k], col + 1);
      f16x2 y;
      if (hh <= G) {  // q or k: RoPE
        float sn, cs;
        sincosf((float)pos * fr[k], &sn, &cs);
        // The QKV epilogue kernel's operations: each FMA written out, rounded to fp32 before the fp16 conversion.
        y = f16x2{static_cast<f16>(as_f32_value(fmaf(x0, cs, -(x1 * sn)))),
                  static_cast<f16>(as_f32_value(fmaf(x0, sn, x1 * cs)))};
      } else {
        y = f16x2{static_cast<f16>(x0), static_cast<f16>(x1)};
      }
      f16* dst = hh < G ? &sm_q[hh][2 * i] : (hh == G ? &sm_kn[2 * i] : &sm_vn[2 * i]);
      *reinterpret_cast<f16x2*>(dst) = y;
    }
  };

  // The first block's K/V do not depend on q: issue them before the workgroup barrier
  // and the fused prologue's arithmetic.  A wavefront without a block of its own loads
  // block b0 and drops it.
  Blk A;
  int blk = b0 + wave;
  if (b0 < b1) {  // uniform: pg0 .. pg1 - 1 and block b0 exist
    const int ptv = ptrow[pg0 + min((int)threadIdx.x, pg1 - pg0 - 1)];
    load_block(A, blk < b1 ? blk : b0);
    // Every thread writes (entries past the split's pages are never read): a store under
    // a condition would let the compiler sink the load below the block's loads.
    sm_pt[threadIdx.x] = ptv;
    if constexpr (FUSED) prologue();
  } else if (writer) {
    prologue();
  }
  if constexpr (FUSED) {
    __syncthreads();  // publishes q, the new k and v and the page-table cache
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const f16x8 v = *reinterpret_cast<const f16x8*>(&sm_q[li < G ? li : 0][8 * lg + 32 * s]);
      qa[s] = (li < G) ? v : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  } else if (pt_cached) {
    __syncthreads();  // publishes the page-table cache
  }
  pt_ready = true;

  float m[4], lsum[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m[r] = -INFINITY;
    lsum[r] = 0.f;
  }
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

  // Scores of block `blk`: sc[j][r] = S[head 4*lg + r][token tb + 16*j + li] (log2 units).
  auto scores = [&](const Blk& o, int blk, f32x4 (&sc)[kTiles]) __attribute__((always_inline)) {
    const int tb = blk * kBlock;
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], o.k[j][s], c, 0, 0, 0);
      const bool valid = tb + 16 * j + li < L;
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[j][r] = valid ? c[r] * scale_log2 : -INFINITY;
    }
  };
  // Online softmax update with the block's scores, then O += P V.
  auto softmax_pv = [&](const Blk& o, f32x4 (&sc)[kTiles]) __attribute__((always_inline)) {
    float alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float bm = sc[0][r];
#pragma unroll
      for (int j = 1; j < kTiles; ++j) bm = fmaxf(bm, sc[j][r]);
      bm = row16_max(bm);
      const float mn = fmaxf(m[r], bm);  // finite: token tb is always visible
      // hardware exp2 (the library exp2f adds range steps that only matter below 2^-126, where p rounds to 0 in fp16):
      // config-4 attention 48.6 -> 47.8 us, config 5 203.7 -> 199.4 (two alternated bench runs on one box)
      alpha[r] = __builtin_amdgcn_exp2f(m[r] - mn);
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < kTiles; ++j) {
        // P V takes p in fp16 (two heads per shuffled dword); l sums the same rounded p.
        const float p = static_cast<float>(static_cast<f16>(__builtin_amdgcn_exp2f(sc[j][r] - mn)));
        sc[j][r] = p;
        ps += p;
      }
      lsum[r] = lsum[r] * alpha[r] + ps;
      m[r] = mn;
    }
    // fp16 p of heads (4g, 4g+1) and (4g+2, 4g+3), g = lane / 16, packed for the shuffles.
    uint32_t pk[kTiles][2];
#pragma unroll
    for (int j = 0; j < kTiles; ++j)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const f16x2 two = {static_cast<f16>(sc[j][2 * q]), static_cast<f16>(sc[j][2 * q + 1])};
        pk[j][q] = __builtin_bit_cast(uint32_t, two);
      }
    // Rescale O, then O += P V.  Head h's alpha / p live in lanes 16*(h/4).., register h%4.
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float a = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha[h & 3]), 16 * (h >> 2)));  // uniform
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= a;
    }
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int tok = 4 * u + lg;
        float vf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = static_cast<float>(o.v[j][u][e]);
#pragma unroll
        for (int h2 = 0; h2 < (G + 1) / 2; ++h2) {
          const uint32_t pp = static_cast<uint32_t>(__shfl(static_cast<int>(pk[j][h2 & 1]), tok + 16 * (h2 >> 1), 64));
          const f16x2 p2 = __builtin_bit_cast(f16x2, pp);
          const float p0 = static_cast<float>(p2.x), p1 = static_cast<float>(p2.y);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[2 * h2][e] = fmaf(p0, vf[e], acc[2 * h2][e]);
          if (2 * h2 + 1 < G) {
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[2 * h2 + 1][e] = fmaf(p1, vf[e], acc[2 * h2 + 1][e]);
          }
        }
      }
    }
  };

  // Register patch of the new token (fused): every tile whose rows include it -- its
  // own and any past-the-end tile re-reading the block's first tile -- takes the k row
  // (lanes li == row) and the v row (lanes lg == row % 4, element row / 4).  Selects,
  // not conditional writes: registers take no runtime index.
  auto patch_k = [&](Blk& o, int blk) __attribute__((always_inline)) {
    const int tb = blk * kBlock;
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const int r = pos - ((tb + 16 * j < L) ? tb + 16 * j : tb);
      const bool hit = r >= 0 && r < 16 && li == r;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f16x8 n = *reinterpret_cast<const f16x8*>(&sm_kn[32 * s + 8 * lg]);
        o.k[j][s] = hit ? n : o.k[j][s];
      }
    }
  };
  auto patch_v = [&](Blk& o, int blk) __attribute__((always_inline)) {
    const int tb = blk * kBlock;
#pragma unroll
    for (int j = 0; j < kTiles; ++j) {
      const int r = pos - ((tb + 16 * j < L) ? tb + 16 * j : tb);
      const bool hit = r >= 0 && r < 16 && lg == (r & 3);
      const f16x8 n = *reinterpret_cast<const f16x8*>(&sm_vn[8 * li]);
#pragma unroll
      for (int u = 0; u < 4; ++u) o.v[j][u] = (hit && u == (r >> 2)) ? n : o.v[j][u];
    }
  };

  // Rotating pipeline: the next block's K is loaded into the K registers as soon as
  // this block's scores have read them, and its V once P V has read this block's V,
  // so every wavefront keeps loads in flight while it computes.  The last block is
  // peeled off, which keeps the steady-state loads unconditional (load counters
  // retire in order; a conditional load would make every wait a full drain).
  {
    const int nb = blk < b1 ? (b1 - blk + kWaves - 1) / kWaves : 0;
    if (nb > 0) {
      // The block holding a fused call's new token (its wavefront in the writer split):
      // its k and v rows are patched into the registers.
      const int blk_new = pos / kBlock;
      const int patch_blk = (writer && blk_new >= b0 && blk_new < b1 && (blk_new - b0) % kWaves == wave) ? blk_new : -1;
      f32x4 sc[kTiles];
      for (int t = 0; t + 1 < nb; ++t, blk += kWaves) {
        if (blk == patch_blk) patch_k(A, blk);
        scores(A, blk, sc);
        load_k(A, blk + kWaves);
        __builtin_amdgcn_sched_barrier(0);
        if (blk == patch_blk) patch_v(A, blk);
        softmax_pv(A, sc);
        load_v(A, blk + kWaves);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (blk == patch_blk) {
        patch_k(A, blk);
        patch_v(A, blk);
      }
      scores(A, blk, sc);
      softmax_pv(A, sc);
    }
  }

  // Wavefront totals: O over the 4 token groups (row k of each 4-value sum holds
  // acc[h][4 * half + k], so every lane writes one), l over the 16 lanes of a row.
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const float v[4] = {acc[h][4 * half], acc[h][4 * half + 1], acc[h][4 * half + 2], acc[h][4 * half + 3]};
      sm_o[wave][h][8 * li + 4 * half + lg] = rows_sum4(v);
    }
#pragma unroll
  for (int r = 0; r < 4; ++r) lsum[r] = row16_sum(lsum[r]);

  if (li == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sm_m[wave][4 * lg + r] = m[r];
      sm_l[wave][4 * lg + r] = lsum[r];
    }
  }
  __syncthreads();

  // Merge the wavefronts: one thread per (head, dim).
  for (int idx = threadIdx.x; idx < G * D; idx += 64 * kWaves) {
    const int h = idx / D, d = idx - h * D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float den = 0.f, o = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = exp2f(sm_m[w][h] - M);
        den = fmaf(sm_l[w][h], f, den);
        o = fmaf(sm_o[w][h][d], f, o);
      }
    }
    const int head = kvh * G + h;
    if (S == 1) {
      out[((size_t)row * Hq + head) * D + d] = static_cast<f16>(den > 0.f ? o / den : 0.f);
    } else {
      part_o[(((size_t)row * Hq + head) * S + split) * D + d] = o;
      if (d == 0) {
        float* ml = part_ml + (((size_t)row * Hq + head) * S + split) * 2;
        ml[0] = M;
        ml[1] = den;
      }
    }
  }
  if (writer && (int)threadIdx.x < kHalf) {  // the KV append (fused): k and v pair t, whole rows
    const int page_idx = pos / P;
    const int slot = page_idx < max_pages ? ptrow[page_idx] : -1;
    if (slot >= 0) {
      const size_t at = (((size_t)slot * Hkv + kvh) * P + (pos - page_idx * P)) * D + 2 * threadIdx.x;
      *reinterpret_cast<uint32_t*>(kp + at) = *reinterpret_cast<const uint32_t*>(&sm_kn[2 * threadIdx.x]);
      *reinterpret_cast<uint32_t*>(vp + at) = *reinterpret_cast<const uint32_t*>(&sm_vn[2 * threadIdx.x]);
    }
  }
}

// ----------------------------------------------------------------------------
// Prefill (q_len > 1), fp16 pools, head_dim 128, G <= 8.  The query vectors of one
// sequence and KV head (vector v = t * G + g over its q_len new tokens) form 16-vector
// tiles, one per wavefront, kPfWaves per workgroup.  A workgroup walks the 32-token
// K/V blocks its last token sees, kPfGroup blocks at a time: every K and V load of a
// group is issued at once, while the previous group is being multiplied, and lands in
// LDS (V transposed) in the other of two buffers.  Each block is read once per 128 query
// vectors instead of once per query row.  Both products run on MFMA 16x16x32 f16:
//   * S^T = K Q^T: A = 16 token rows of K (lane t + 16g holds K[t][32s + 8g ..]), B =
//     Q^T (lane q + 16g holds Q[q][32s + 8g ..]); lane q + 16g ends with S[q][4g + r]
//     of each 16-token tile;
//   * O^T = V^T P^T: the B operand is P as the lanes already hold it -- lane q + 16g
//     takes P[q][4g .. 4g+3] of tile 0 and P[q][16 + 4g .. +3] of tile 1 as its 8 k
//     values -- and V^T's A operand takes the same token order (lane d + 16g: V^T[d] at
//     tokens 4g .. and 16 + 4g ..), so no lane exchange is needed; lane q + 16g ends with
//     O[q][16 dt + 4g + r], all of one query, so the softmax rescale and the final 1/l
//     are per lane (O = P V, the other way round, spread four queries over each lane and
//     needed four shuffles of the rescale factors per block).
// Causal mask per query vector (keys at positions <= its token's), applied only to the
// blocks a wavefront's first query does not see whole; softmax as in the decode kernel
// (base 2, p rounded to fp16, l summing the rounded p), with the hardware exp2 (the
// library exp2f's extra range steps only change results below 2^-126, which round to
// zero in fp16 p and are negligible in the rescale), and the rescale of O skipped when
// no lane's running max moved.  A wavefront skips the blocks past its last token.  The
// tiles of a sequence are dispatched last first, so the longest contexts start first.
// At two blocks per LDS buffer a workgroup holds 70 KiB and 112 VGPRs, so two fit on a
// CU.  Against one workgroup per CU at four blocks per buffer (140 KiB), the library
// exp2f, O = P V and V^T written 4 tokens x 16 column chunks per wavefront (4 banks), a
// 2048-token prompt (32/8 heads) took 135 against 224 us, 4 x 512 tokens 44 against 66.
// PAIRED: once the one-tile grid fills both workgroup slots of every CU, all of it is
// resident at once and the longest tiles set the kernel's time (at 2048 tokens tile 63
// walks 64 blocks, the mean is 32.5).  A workgroup then runs tile tiles - 1 - x and tile
// x one after the other (tiles + 1 tiles' worth of blocks each, 120 VGPRs): 2048 tokens
// 121 us, 4096 tokens 308 against 401, 8 x 512 tokens 60 against 80, the same bits.
// Smaller grids keep one tile per workgroup.  NG: blocks per LDS buffer.  A grid of at
// most one workgroup per CU takes 4 (143 KiB; 166 VGPRs paired, 129 not), twice the loads
// in flight: 2048 tokens 110 us, 2 x 1024 61 against 67, 2 x 512 28.1 against 29.2; a
// larger one would then run in two rounds (4096 tokens 374 against 289), so it keeps 2.
constexpr int kPfWaves = 8;
constexpr int kPfGroup = 2;    // blocks per LDS buffer (two buffers: 70 KiB)
constexpr int kPfKRow = 136;   // K row stride in LDS (halves): 256 B + 16, a tile's rows on distinct banks
constexpr int kPfVRow = 36;    // V^T row stride (halves): 64 B + 8; V is loaded 32 tokens x 2 column chunks per
                               // wavefront, so each transposed 2-byte write covers 32 banks

template <bool PAIRED, int NG>
__global__ __launch_bounds__(64 * kPfWaves) void attn_prefill_f16_d128(
    const f16* __restrict__ q, const f16* __restrict__ kp, const f16* __restrict__ vp,
    const int32_t* __restrict__ pt, const int32_t* __restrict__ lens, f16* __restrict__ out, int q_len, int Hq,
    int Hkv, int P, int max_pages, float scale_log2) {
  constexpr int D = 128;
  static_assert(kBlock == 32 && 64 * kPfWaves == kBlock * (D / 8), "one 16-byte K and V chunk per thread");
  static_assert(NG == kPfGroup || NG == 2 * kPfGroup, "blocks per LDS buffer");
  __shared__ __align__(16) f16 sk[2][NG][kBlock * kPfKRow];
  __shared__ __align__(16) f16 sv[2][NG][D * kPfVRow];
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int G = Hq / Hkv;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int nvec = q_len * G;
  const int max_ctx = max_pages * P;
  const int L = lens[b];
  const int Lc = min(L, max_ctx);  // keys the page table can address
  const int past = L - q_len;      // context before the new tokens
  const int32_t* ptrow = pt + (size_t)b * max_pages;
  // Last key position query vector v sees (negative: none, its output is zero).
  auto pos_of = [&](int v) __attribute__((always_inline)) { return min(past + v / G, Lc - 1); };
  const int tiles = (nvec + 16 * kPfWaves - 1) / (16 * kPfWaves);
  // Unpaired: one tile per workgroup, the last (longest) tiles first.  Paired: tile tiles - 1 - x, then tile x
  // (once when they coincide), so every workgroup walks tiles + 1 tiles' worth of blocks under the causal mask.
  for (int pass = 0; pass < (PAIRED ? 2 : 1); ++pass) {
    const int tile = !PAIRED ? (int)(gridDim.x - 1 - blockIdx.x)
                             : (pass == 0 ? tiles - 1 - (int)blockIdx.x : (int)blockIdx.x);
    if (PAIRED && pass == 1) {
      if (tile == tiles - 1 - (int)blockIdx.x) break;
      __syncthreads();  // the first tile's LDS reads are done before the second's first stash
    }
    const int tv0 = tile * 16 * kPfWaves;                     // the workgroup's first vector
    const int tv1 = min(nvec, tv0 + 16 * kPfWaves) - 1;       // and its last
    const int nblk = pos_of(tv1) >= 0 ? pos_of(tv1) / kBlock + 1 : 0;  // blocks the last token sees
    const int v0 = tv0 + 16 * wave;                           // this wavefront's first vector
    const int wlast = min(nvec - 1, v0 + 15);
    const int wblk = (v0 < nvec && pos_of(wlast) >= 0) ? pos_of(wlast) / kBlock + 1 : 0;  // uniform

    // Thread t loads 16 bytes of K and of V per block: K at token t / 16, dims 8 * (t % 16); V at token t % 32,
    // dims 8 * (t / 32).
    const int lt = threadIdx.x >> 4, lc = threadIdx.x & 15;
    const int vt = threadIdx.x & 31, vc = threadIdx.x >> 5;
    f16x8 kr[NG], vr[NG];
    auto load_group = [&](int g0, int nb) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        if (i < nb) {
          const int tok = min((g0 + i) * kBlock + lt, Lc - 1);  // past the context: masked, a valid page
          const int page = ptrow[tok / P];
          const size_t at = (((size_t)page * Hkv + kvh) * P + tok % P) * D + 8 * lc;
          kr[i] = *reinterpret_cast<const f16x8*>(kp + at);
          const int vtok = min((g0 + i) * kBlock + vt, Lc - 1);
          const int vpage = ptrow[vtok / P];
          vr[i] = *reinterpret_cast<const f16x8*>(vp + (((size_t)vpage * Hkv + kvh) * P + vtok % P) * D + 8 * vc);
        }
      }
    };
    auto stash_group = [&](int buf, int nb) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NG; ++i) {
        if (i < nb) {
          *reinterpret_cast<f16x8*>(&sk[buf][i][lt * kPfKRow + 8 * lc]) = kr[i];
#pragma unroll
          for (int e = 0; e < 8; ++e) sv[buf][i][(8 * vc + e) * kPfVRow + vt] = vr[i][e];
        }
      }
    };
    if (nblk > 0) load_group(0, min(NG, nblk));

    // Q^T as the B operand (zero past the last vector), and each lane's query position.
    f16x8 qb[4];
    const int vq = v0 + li;
    const bool live = vq < nvec;
    const int qpos = pos_of(live ? vq : nvec - 1);
    const int qmin = pos_of(min(v0, nvec - 1));  // the wavefront's first query position (the least)
    {
      const int vv = live ? vq : 0;
      const int t = vv / G, g = vv - t * G;
      const f16* qrow = q + (((size_t)b * q_len + t) * Hq + (size_t)kvh * G + g) * D + 8 * lg;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f16x8 x = *reinterpret_cast<const f16x8*>(qrow + 32 * s);
        qb[s] = live ? x : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
    if (nblk > 0) stash_group(0, min(NG, nblk));
    __syncthreads();

    float m = -INFINITY, l = 0.f;  // query li: running max (every lane of the query), this lane's share of the sum
    f32x4 acc[D / 16];             // O[query 4 lg + r][16 dt + li]
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto block = [&](int buf, int i, int blk) __attribute__((always_inline)) {
      f32x4 c[kTiles];
#pragma unroll
      for (int j = 0; j < kTiles; ++j) {
        c[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const f16x8 a = *reinterpret_cast<const f16x8*>(&sk[buf][i][(16 * j + li) * kPfKRow + 32 * s + 8 * lg]);
          c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qb[s], c[j], 0, 0, 0);
        }
      }
      float mx = -INFINITY;
      if (blk * kBlock + kBlock - 1 <= qmin) {  // uniform: every query of the wavefront sees the whole block
#pragma unroll
        for (int j = 0; j < kTiles; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            c[j][r] = c[j][r] * scale_log2;
            mx = fmaxf(mx, c[j][r]);
          }
      } else {
#pragma unroll
        for (int j = 0; j < kTiles; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int key = blk * kBlock + 16 * j + 4 * lg + r;
            c[j][r] = key <= qpos ? c[j][r] * scale_log2 : -INFINITY;
            mx = fmaxf(mx, c[j][r]);
          }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // Block 0 comes first and key 0 is visible to every query with a position, so m is finite from then on and
      // a fully masked later block leaves mn = m, alpha = 1 and p = 0.  A query with no key at all keeps m = -inf:
      // alpha 1 and p 0 (not the NaN of -inf - -inf), l stays 0 and its output 0.
      const float mn = fmaxf(m, mx);
      const bool none = mn == -INFINITY;
      const float alpha = none ? 1.f : __builtin_amdgcn_exp2f(m - mn);
      f16x8 pa;
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < kTiles; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const f16 p = static_cast<f16>(none ? 0.f : __builtin_amdgcn_exp2f(c[j][r] - mn));
          pa[4 * j + r] = p;
          ps += static_cast<float>(p);
        }
      l = l * alpha + ps;
      m = mn;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {  // uniform
#pragma unroll
        for (int dt = 0; dt < D / 16; ++dt) acc[dt] *= alpha;
      }
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        const f16* vrow = &sv[buf][i][(16 * dt + li) * kPfVRow];
        const f16x4 lo = *reinterpret_cast<const f16x4*>(vrow + 4 * lg);
        const f16x4 hi = *reinterpret_cast<const f16x4*>(vrow + 16 + 4 * lg);
        const f16x8 vb = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb, pa, acc[dt], 0, 0, 0);
      }
    };
    int buf = 0;
    for (int g0 = 0; g0 < nblk; g0 += NG, buf ^= 1) {  // uniform
      const int nb = min(NG, nblk - g0);
      const int g1 = g0 + NG, nb1 = min(NG, nblk - g1);
      if (nb1 > 0) load_group(g1, nb1);  // in flight during this group's math
      for (int i = 0; i < nb; ++i)
        if (g0 + i < wblk) block(buf, i, g0 + i);
      if (nb1 > 0) stash_group(buf ^ 1, nb1);
      __syncthreads();
    }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);

    if (live) {
      const int t = vq / G, g = vq - t * G;
      f16* po = out + (((size_t)b * q_len + t) * Hq + (size_t)kvh * G + g) * D + 4 * lg;
      const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt)
        *reinterpret_cast<f16x4*>(po + 16 * dt) = f16x4{static_cast<f16>(acc[dt][0] * inv), static_cast<f16>(acc[dt][1] * inv),
                                                      static_cast<f16>(acc[dt][2] * inv), static_cast<f16>(acc[dt][3] * inv)};
    }
  }  // pass
}

// ----------------------------------------------------------------------------
// Generic VALU kernel (fp32 or fp16 pools, any page size, head_dim <= 256):
// one wavefront per (128-token chunk, KV head, row); always writes partials.
template <typename T>
__global__ __launch_bounds__(64) void attn_chunk_generic(
    const T* __restrict__ q, const T* __restrict__ kp, const T* __restrict__ vp,
    const int32_t* __restrict__ pt, const int32_t* __restrict__ lens,
    float* __restrict__ part_o, float* __restrict__ part_ml,
    int q_len, int Hq, int Hkv, int D, int P, int max_pages, int NC, float scale_log2) {
  __shared__ float qs[256];
  __shared__ float ps[kChunk];
  const int chunk = blockIdx.x, kvh = blockIdx.y, row = blockIdx.z;
  const int L = visible_len(lens, row, q_len, max_pages * P);
  const int t0 = chunk * kChunk;
  const int G = Hq / Hkv;
  const int lane = threadIdx.x;
  const int n = max(0, min(L, t0 + kChunk) - t0);
  const int b = row / q_len;
  const int32_t* ptrow = pt + (size_t)b * max_pages;
  for (int h = 0; h < G; ++h) {
    const int head = kvh * G + h;
    float* ml = part_ml + (((size_t)row * Hq + head) * NC + chunk) * 2;
    if (n == 0) {  // empty chunk: neutral partial
      for (int d = lane; d < D; d += 64) part_o[(((size_t)row * Hq + head) * NC + chunk) * D + d] = 0.f;
      if (lane == 0) {
        ml[0] = -INFINITY;
        ml[1] = 0.f;
      }
      continue;
    }
    __syncthreads();
    for (int d = lane; d < D; d += 64) qs[d] = to_f32(q[((size_t)row * Hq + head) * D + d]);
    __syncthreads();
    float mx = -INFINITY;
    for (int j = lane; j < n; j += 64) {
      const int t = t0 + j;
      const int page = ptrow[t / P];
      const T* krow = kp + (((size_t)page * Hkv + kvh) * P + (t % P)) * D;
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot = fmaf(qs[d], to_f32(krow[d]), dot);
      const float s = dot * scale_log2;
      ps[j] = s;
      mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    float sum = 0.f;
    for (int j = lane; j < n; j += 64) {
      const float p = exp2f(ps[j] - mx);
      ps[j] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    __syncthreads();
    for (int d = lane; d < D; d += 64) {
      float o = 0.f;
      for (int j = 0; j < n; ++j) {
        const int t = t0 + j;
        const int page = ptrow[t / P];
        o = fmaf(ps[j], to_f32(vp[(((size_t)page * Hkv + kvh) * P + (t % P)) * D + d]), o);
      }
      part_o[(((size_t)row * Hq + head) * NC + chunk) * D + d] = o;
    }
    if (lane == 0) {
      ml[0] = mx;
      ml[1] = sum;
    }
  }
}

// ----------------------------------------------------------------------------
// Merge S partials of one (row, head): out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
// Latency-bound (a few KiB per workgroup), so no load waits for another: thread s
// reads split s's (m, l), the weights 2^(m_s - M) go through LDS, and each output
// element's S partials are loaded 8 at a time before they are summed.  Sums run in
// split order, as the serial form for S > kMergeFast does.  o * inv is rounded to fp32
// before the fp16 conversion (as_f32_value: no single-rounding mixed-precision multiply),
// the same two roundings the O projection's merge (qgemm.hip, attn_merged_chunk) makes.
constexpr int kMergeFast = 128;
template <typename T>
__global__ __launch_bounds__(128) void attn_merge(const float* __restrict__ part_o, const float* __restrict__ part_ml,
                                                  T* __restrict__ out, int Hq, int D, int S) {
  const int head = blockIdx.x, row = blockIdx.y;
  const float* ml = part_ml + ((size_t)row * Hq + head) * S * 2;
  if (S <= kMergeFast) {
    __shared__ float sw[kMergeFast], sl[kMergeFast], smax[2];
    const int t = threadIdx.x;
    const float mv = t < S ? ml[2 * t] : -INFINITY;
    const float lv = t < S ? ml[2 * t + 1] : 0.f;
    const float wm = wave_max(mv);
    if ((t & 63) == 0) smax[t >> 6] = wm;
    __syncthreads();
    const float M = fmaxf(smax[0], smax[1]);
    sw[t] = (t < S && M != -INFINITY) ? exp2f(mv - M) : 0.f;
    sl[t] = lv;
    __syncthreads();
    float den = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < S; ++s) den = fmaf(sl[s], sw[s], den);
    const float inv = den > 0.f ? 1.f / den : 0.f;
    const float* po = part_o + ((size_t)row * Hq + head) * S * D;
    for (int d = t; d < D; d += 128) {
      float o = 0.f;
      for (int s0 = 0; s0 < S; s0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = po[(size_t)min(s0 + j, S - 1) * D + d];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (s0 + j < S) o = fmaf(v[j], sw[s0 + j], o);
      }
      out[((size_t)row * Hq + head) * D + d] = from_f32<T>(as_f32_value(o * inv));
    }
    return;
  }
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, ml[2 * s]);
  float den = 0.f;
  if (M != -INFINITY)
    for (int s = 0; s < S; ++s) den = fmaf(ml[2 * s + 1], exp2f(ml[2 * s] - M), den);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  const float* po = part_o + ((size_t)row * Hq + head) * S * D;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float o = 0.f;
    if (M != -INFINITY)
      for (int s = 0; s < S; ++s) o = fmaf(po[(size_t)s * D + d], exp2f(ml[2 * s] - M), o);
    out[((size_t)row * Hq + head) * D + d] = from_f32<T>(as_f32_value(o * inv));
  }
}

int max_splits(int max_context) { return max(1, (max_context + kMinSplitTokens - 1) / kMinSplitTokens); }

int generic_chunks(int max_context) { return max(1, (max_context + kChunk - 1) / kChunk); }

// Splits for the fp16 path: about one workgroup per CU (256 / (rows * kv_heads)),
// at most 8.  Measured at 2048 tokens of context, 32/8 heads (attention + merge):
// batch 1 best at 8 splits (13.1 us; 16 splits 14.8, 64 splits 34), batch 4 at 4-8,
// batch 8 at 4 (19.7 us; 8 splits 25.3), batch 16 at 2 (29.5 us; 1 split 32.8,
// 4 splits 33.9), batch 32 at 1.  More splits add per-workgroup fixed cost (page
// table, q, first load latency, the 8-wavefront merge) and a longer merge.
int choose_splits(int rows, int Hkv, int max_context) {
  const long groups = (long)rows * Hkv;
  const int want = (int)min(8L, max(1L, 256 / groups));
  return max(1, min(want, max_splits(max_context)));
}

// The MFMA kernel serves fp16 pools with head_dim 128, pages of a multiple of 16
// tokens and up to 8 query heads per KV head; everything else runs the generic kernel.
bool mfma_path(int kv_dtype, int D, int P, int G) { return kv_dtype == CIR_F16 && D == 128 && P % 16 == 0 && G <= 8; }

// Context splits of a launch: about one workgroup per CU on the MFMA path, one
// partial per 128-token chunk on the generic path.
int launch_splits(int rows, int Hkv, int max_ctx, bool mfma) {
  return mfma ? choose_splits(rows, Hkv, max_ctx) : generic_chunks(max_ctx);
}

// Bytes of split partials (O, then (max, sum)) a launch writes: none when the MFMA
// kernel runs unsplit and writes the output itself.
size_t partial_bytes(int rows, int Hq, int D, int S, bool mfma) {
  if (mfma && S == 1) return 0;
  return (size_t)rows * Hq * S * ((size_t)D + 2) * sizeof(float);
}

// Compute units of the current device, looked up once per device.
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int launch_attention(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                     const int32_t* seq_lens, void* out, void* workspace, size_t workspace_bytes,
                     int batch, int q_len, int Hq, int Hkv, int D, int P, int max_pages, float scale,
                     int kv_dtype, void* stream, QkvIn qkv = QkvIn{nullptr, 0, nullptr, nullptr},
                     bool merge = true, bool exact_workspace = false) {
  CIR_CHECK_ARG(batch >= 0 && q_len >= 1, "attention: batch must be >= 0 and q_len >= 1");
  if (batch == 0) return 0;
  CIR_CHECK_ARG((q || qkv.part) && k_pool && v_pool && page_table && seq_lens && out, "attention: null pointer");
  CIR_CHECK_ARG(Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attention: num_heads (%d) must be a multiple of num_kv_heads (%d)", Hq, Hkv);
  CIR_CHECK_ARG(D > 0 && D <= 256, "attention: head_dim %d out of range (1..256)", D);
  CIR_CHECK_ARG(P > 0 && max_pages > 0, "attention: page_size and max_pages must be positive");
  CIR_CHECK_ARG(kv_dtype == CIR_F16 || kv_dtype == CIR_F32, "attention: kv_dtype must be CIR_F16 or CIR_F32");
  const int rows = batch * q_len;
  const int max_ctx = max_pages * P;
  CIR_CHECK_ARG(rows <= 65535 && Hkv <= 65535, "attention: grid too large");
  const float scale_log2 = scale * kLog2e;
  const int G = Hq / Hkv;
  hipStream_t s = as_stream(stream);
  const bool mfma = mfma_path(kv_dtype, D, P, G);
  const int S = launch_splits(rows, Hkv, max_ctx, mfma);
  // The advertised size (cir_paged_attention_workspace_bytes) covers any split count;
  // the static-scratch entry point checks the bytes this launch writes instead.
  const size_t need = exact_workspace ? partial_bytes(rows, Hq, D, S, mfma)
                                      : cir_paged_attention_workspace_bytes(rows, Hq, D, max_ctx);
  CIR_CHECK_ARG(workspace && workspace_bytes >= need, "attention: workspace too small (%zu < %zu)", workspace_bytes,
                need);
  CIR_CHECK_ARG(!qkv.part || (mfma && q_len == 1 && qkv.splits >= 1 && qkv.inv_freq && qkv.positions),
                "attention: the fused QKV input needs decode (q_len 1), fp16 pools, head_dim 128, page_size %% 16 == 0, "
                "num_heads/num_kv_heads <= 8 and inv_freq/positions");
  CIR_CHECK_ARG(merge || (mfma && S > 1), "attention: unmerged partials need the fp16 decode path with > 1 split");
  float* part_o = static_cast<float*>(workspace);
  float* part_ml = part_o + (size_t)rows * Hq * S * D;
  dim3 grid(S, Hkv, rows);
  if (mfma && q_len > 1) {  // prefill: query tiles of 128 vectors over each sequence's blocks, no partials
    const int tiles = (q_len * G + 16 * kPfWaves - 1) / (16 * kPfWaves);
    // Pairs of tiles per workgroup once the unpaired grid fills every CU's two workgroup slots: the causal
    // mask's long and short tiles then share a workgroup instead of the longest setting the kernel's time.
    const long one_tile = (long)tiles * Hkv * batch;
    const bool paired = tiles > 1 && one_tile >= 2L * device_cus();
    const long workgroups = paired ? (long)((tiles + 1) / 2) * Hkv * batch : one_tile;
    // A grid of at most one workgroup per CU stages twice the blocks per buffer (143 KiB of LDS, twice the loads
    // in flight); a larger one keeps 70 KiB so two workgroups share a CU and the grid runs in one round.
    const bool deep = workgroups <= device_cus();
    const auto kernel = paired ? (deep ? attn_prefill_f16_d128<true, 2 * kPfGroup> : attn_prefill_f16_d128<true, kPfGroup>)
                               : (deep ? attn_prefill_f16_d128<false, 2 * kPfGroup>
                                       : attn_prefill_f16_d128<false, kPfGroup>);
    kernel<<<dim3(paired ? (tiles + 1) / 2 : tiles, Hkv, batch), 64 * kPfWaves, 0, s>>>(
        static_cast<const f16*>(q), static_cast<const f16*>(k_pool), static_cast<const f16*>(v_pool), page_table,
        seq_lens, static_cast<f16*>(out), q_len, Hq, Hkv, P, max_pages, scale_log2);
    return launch_status();
  }
  if (mfma) {
    // Longest rows first when the workgroups outnumber the CUs (they then run in rounds).
    const int sort_rows = q_len == 1 && rows <= 64 * kWaves && (long)S * Hkv * rows > device_cus();
    auto kq = static_cast<const f16*>(q);
    auto kk = static_cast<f16*>(const_cast<void*>(k_pool));
    auto kv = static_cast<f16*>(const_cast<void*>(v_pool));
    auto ko = static_cast<f16*>(out);
#define CIR_ATT_CASE(g)                                                                                             \
  case g:                                                                                                           \
    if (qkv.part)                                                                                                   \
      attn_f16_d128<g, true><<<grid, 64 * kWaves, 0, s>>>(kq, kk, kv, page_table, seq_lens, ko, part_o, part_ml,   \
                                                           q_len, Hq, Hkv, P, max_pages, S, scale_log2,          \
                                                           sort_rows, qkv);                                        \
    else                                                                                                            \
      attn_f16_d128<g, false><<<grid, 64 * kWaves, 0, s>>>(kq, kk, kv, page_table, seq_lens, ko, part_o, part_ml,  \
                                                            q_len, Hq, Hkv, P, max_pages, S, scale_log2,         \
                                                            sort_rows, qkv);                                       \
    break;
    switch (G) {
      CIR_ATT_CASE(1) CIR_ATT_CASE(2) CIR_ATT_CASE(3) CIR_ATT_CASE(4)
      CIR_ATT_CASE(5) CIR_ATT_CASE(6) CIR_ATT_CASE(7) CIR_ATT_CASE(8)
    }
#undef CIR_ATT_CASE
    const int st = launch_status();
    if (st || S == 1 || !merge) return st;
  } else {
    if (kv_dtype == CIR_F16) {
      attn_chunk_generic<f16><<<grid, 64, 0, s>>>(static_cast<const f16*>(q), static_cast<const f16*>(k_pool),
                                                  static_cast<const f16*>(v_pool), page_table, seq_lens, part_o,
                                                  part_ml, q_len, Hq, Hkv, D, P, max_pages, S, scale_log2);
    } else {
      attn_chunk_generic<float><<<grid, 64, 0, s>>>(static_cast<const float*>(q), static_cast<const float*>(k_pool),
                                                    static_cast<const float*>(v_pool), page_table, seq_lens, part_o,
                                                    part_ml, q_len, Hq, Hkv, D, P, max_pages, S, scale_log2);
    }
    const int st = launch_status();
    if (st) return st;
  }
  dim3 mgrid(Hq, rows);
  if (kv_dtype == CIR_F16) {
    attn_merge<f16><<<mgrid, 128, 0, s>>>(part_o, part_ml, static_cast<f16*>(out), Hq, D, S);
  } else {
    attn_merge<float><<<mgrid, 128, 0, s>>>(part_o, part_ml, static_cast<float*>(out), Hq, D, S);
  }
  return launch_status();
}

}  // namespace
}  // namespace cir

extern "C" size_t cir_paged_attention_workspace_bytes(int rows, int num_heads, int head_dim, int max_context) {
  if (rows <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  // Partial O and (max, sum) per (row, head, split), sized for the larger split count of the two paths.
  const int a = cir::max_splits(max_context), c = cir::generic_chunks(max_context);
  const size_t s = (size_t)(a > c ? a : c);
  return (size_t)rows * num_heads * s * ((size_t)head_dim + 2) * sizeof(float);
}

extern "C" int cir_paged_decode_attention(const void* q, const void* k_pool, const void* v_pool,
                                          const int32_t* page_table, const int32_t* seq_lens, void* out,
                                          void* workspace, size_t workspace_bytes, int batch, int num_heads,
                                          int num_kv_heads, int head_dim, int page_size, int max_pages, float scale,
                                          int kv_dtype, void* stream) {
  return cir::launch_attention(q, k_pool, v_pool, page_table, seq_lens, out, workspace, workspace_bytes, batch, 1,
                               num_heads, num_kv_heads, head_dim, page_size, max_pages, scale, kv_dtype, stream);
}

extern "C" int cir_paged_decode_splits(int batch, int num_heads, int num_kv_heads, int head_dim, int page_size,
                                       int max_pages, int kv_dtype) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 || page_size <= 0 || max_pages <= 0) return 0;
  const bool mfma = num_heads % num_kv_heads == 0 &&
                    cir::mfma_path(kv_dtype, head_dim, page_size, num_heads / num_kv_heads);
  return cir::launch_splits(batch, num_kv_heads, max_pages * page_size, mfma);
}

extern "C" int cir_paged_prefill_attention(const void* q, const void* k_pool, const void* v_pool,
                                           const int32_t* page_table, const int32_t* seq_lens, void* out,
                                           void* workspace, size_t workspace_bytes, int batch, int q_len,
                                           int num_heads, int num_kv_heads, int head_dim, int page_size,
                                           int max_pages, float scale, int kv_dtype, void* stream) {
  return cir::launch_attention(q, k_pool, v_pool, page_table, seq_lens, out, workspace, workspace_bytes, batch,
                               q_len, num_heads, num_kv_heads, head_dim, page_size, max_pages, scale, kv_dtype,
                               stream);
}

extern "C" int cir_paged_decode_attention_qkv(const float* qkv_partial, int splits, const float* inv_freq,
                                              const int32_t* positions, void* k_pool, void* v_pool,
                                              const int32_t* page_table, const int32_t* seq_lens, void* out,
                                              void* workspace, size_t workspace_bytes, int batch, int num_heads,
                                              int num_kv_heads, int head_dim, int page_size, int max_pages,
                                              float scale, void* stream) {
  CIR_CHECK_ARG(batch == 0 || qkv_partial, "attention_qkv: null qkv_partial");
  return cir::launch_attention(nullptr, k_pool, v_pool, page_table, seq_lens, out, workspace, workspace_bytes, batch,
                               1, num_heads, num_kv_heads, head_dim, page_size, max_pages, scale, CIR_F16, stream,
                               cir::QkvIn{qkv_partial, splits, inv_freq, positions});
}

extern "C" int cir_paged_decode_attention_qkv_parts(const float* qkv_partial, int splits, const float* inv_freq,
                                                    const int32_t* positions, void* k_pool, void* v_pool,
                                                    const int32_t* page_table, const int32_t* seq_lens, void* workspace,
                                                    size_t workspace_bytes, int batch, int num_heads, int num_kv_heads,
                                                    int head_dim, int page_size, int max_pages, float scale,
                                                    void* stream) {
  CIR_CHECK_ARG(batch == 0 || qkv_partial, "attention_qkv_parts: null qkv_partial");
  // `out` is never written on this path; the workspace pointer stands in for the non-null check.
  return cir::launch_attention(nullptr, k_pool, v_pool, page_table, seq_lens, workspace, workspace, workspace_bytes,
                               batch, 1, num_heads, num_kv_heads, head_dim, page_size, max_pages, scale, CIR_F16,
                               stream, cir::QkvIn{qkv_partial, splits, inv_freq, positions}, false);
}


// ----------------------------------------------------------------------------
// Decode attention that allocates nothing (cir_paged_decode_attention_noalloc).
// The split partials go to `scratch`, a device array of fixed size that every call
// on a GPU shares.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol): its device address is looked up once
// per device with hipGetSymbolAddress and kept in g_scratch_ptr.
static constexpr size_t kScratchBytes = CIR_ATTENTION_NOALLOC_MAX_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace cir {
namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first call
// for that device, with that device current).
int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("attention_noalloc: hipGetDevice failed: %s", hipGetErrorString(e));
    return static_cast<int>(e);
  }
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("attention_noalloc: device %d beyond the %d devices the library tracks", dev, kMaxDevices);
    return static_cast<int>(hipErrorInvalidDevice);
  }
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        set_error("attention_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
        return static_cast<int>(e != hipSuccess ? e : hipErrorInvalidSymbol);
      }
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

}  // namespace
}  // namespace cir

extern "C" int cir_paged_decode_attention_noalloc(const void* q, const void* k_pool, const void* v_pool,
                                                  const int32_t* page_table, const int32_t* seq_lens, void* out,
                                                  int batch, int num_heads, int num_kv_heads, int head_dim,
                                                  int page_size, int max_pages, float scale, int kv_dtype,
                                                  void* stream) {
  CIR_CHECK_ARG(batch >= 0, "attention_noalloc: batch must be >= 0");
  if (batch == 0) return 0;
  CIR_CHECK_ARG(num_kv_heads > 0 && num_heads > 0 && num_heads % num_kv_heads == 0,
                "attention_noalloc: num_heads (%d) must be a multiple of num_kv_heads (%d)", num_heads, num_kv_heads);
  CIR_CHECK_ARG(head_dim > 0 && head_dim <= 256, "attention_noalloc: head_dim %d out of range (1..256)", head_dim);
  CIR_CHECK_ARG(page_size > 0 && max_pages > 0, "attention_noalloc: page_size and max_pages must be positive");
  CIR_CHECK_ARG(batch <= 65535, "attention_noalloc: grid too large");
  const bool mfma = cir::mfma_path(kv_dtype, head_dim, page_size, num_heads / num_kv_heads);
  const int S = cir::launch_splits(batch, num_kv_heads, max_pages * page_size, mfma);
  const size_t need = cir::partial_bytes(batch, num_heads, head_dim, S, mfma);
  CIR_CHECK_ARG(need <= kScratchBytes,
                "attention_noalloc: the split partials need %zu bytes, more than the %zu bytes of static scratch "
                "(batch %d, %d heads, head_dim %d, %d splits); use cir_paged_decode_attention with a workspace",
                need, kScratchBytes, batch, num_heads, head_dim, S);
  void* ws = nullptr;
  const int st = cir::scratch_on_current_device(&ws);
  if (st) return st;
  return cir::launch_attention(q, k_pool, v_pool, page_table, seq_lens, out, ws, kScratchBytes, batch, 1, num_heads,
                               num_kv_heads, head_dim, page_size, max_pages, scale, kv_dtype, stream,
                               cir::QkvIn{nullptr, 0, nullptr, nullptr}, true, true);
}
