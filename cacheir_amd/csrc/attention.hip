// Paged decode / prefill attention for gfx950.
//
// Work unit: one wavefront per (row, KV head, 128-token chunk of the context).
// A row is one query token (batch * q_len rows); all GQA query heads of the KV
// head are handled by the same wavefront, so each K/V page is read from HBM once.
//
// fp16 pools, head_dim 128 (Llama-3 / Qwen2 shapes):
//   * S = Q K^T on MFMA 16x16x32 f16: A = the group's query heads padded to 16
//     rows, B = one 16-token tile of K read straight from the page (token rows of
//     256 B, so a wavefront load covers 16 x 64 B); fp32 accumulate.
//   * softmax is exact within the chunk (scores for the whole chunk stay in
//     registers), in base 2 with scale*log2(e) folded into the scores.
//   * O = P V on VALU: each lane owns 8 contiguous head dims of 4 token rows per
//     tile (1 KiB contiguous per load instruction); P is fetched from the score
//     lanes with ds_bpermute shuffles; the four token groups are summed once per
//     chunk with cross-row shuffles.
//   * The chunk's unnormalised O and its (max, sum) go to the workspace; a
//     combine kernel merges the chunks with log-sum-exp weights.
// fp32 pools (tiny-model parity path) use a plain VALU kernel with the same
// workspace layout and the same combine kernel.
//
// Reference semantics: cacheir/backends/triton_kernels.py:174-217 (paged gather
// pool[page_table[b, t // P], kvh, t % P], GQA kvh = h // (Hq/Hkv), positions
// t < seq_len) and cacheir/runtime/cpu.py:342-377 (softmax(q.k * scale) v,
// prefill causal mask).
#include "common.hpp"

#include <math.h>

namespace cir {
namespace {

constexpr int kChunk = 128;          // context tokens per wavefront
constexpr int kTiles = kChunk / 16;  // 16-token MFMA tiles per chunk
constexpr float kLog2e = 1.4426950408889634f;

// Tokens visible to query row `row`, clamped to what the page table can address.
__device__ __forceinline__ int visible_len(const int32_t* lens, int row, int q_len, int max_ctx) {
  const int b = row / q_len;
  const int s = row - b * q_len;
  return min(lens[b] - q_len + s + 1, max_ctx);
}

// Merge the chunks of heads [head0, head0 + nh) of one row:
// out = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.  One wavefront.
template <typename T>
__device__ void merge_chunks(const float* __restrict__ part_o, const float* __restrict__ part_ml, T* __restrict__ out,
                             int row, int head0, int nh, int Hq, int D, int NC, int nc, int lane) {
  for (int h = 0; h < nh; ++h) {
    const int head = head0 + h;
    const float* ml = part_ml + ((size_t)row * Hq + head) * NC * 2;
    float M = -INFINITY;
    for (int c = 0; c < nc; ++c) M = fmaxf(M, ml[2 * c]);
    float denom = 0.f;
    for (int c = 0; c < nc; ++c) denom += ml[2 * c + 1] * exp2f(ml[2 * c] - M);
    const float inv = denom > 0.f ? 1.f / denom : 0.f;
    const float* po = part_o + ((size_t)row * Hq + head) * NC * D;
    for (int d = lane; d < D; d += 64) {
      float o = 0.f;
      for (int c = 0; c < nc; ++c) o = fmaf(po[(size_t)c * D + d], exp2f(ml[2 * c] - M), o);
      out[((size_t)row * Hq + head) * D + d] = from_f32<T>(o * inv);
    }
  }
}

// Called by every wavefront after it stored its chunk.  The wavefront that takes the
// last ticket of (row, kvh) merges all chunks and resets the counter to zero.
template <typename T>
__device__ void finish_chunk(const float* part_o, const float* part_ml, int* counters, T* out, int row, int kvh,
                             int G, int Hq, int Hkv, int D, int NC, int L, int lane) {
  __threadfence();  // publish this chunk's partials (agent-scope release)
  int ticket = 0;
  if (lane == 0) ticket = atomicAdd(&counters[(size_t)row * Hkv + kvh], 1);
  ticket = __shfl(ticket, 0, 64);
  const int nc = (L + kChunk - 1) / kChunk;
  if (ticket != nc - 1) return;
  __threadfence();  // acquire: see every other chunk's partials
  merge_chunks<T>(part_o, part_ml, out, row, kvh * G, G, Hq, D, NC, nc, lane);
  if (lane == 0) counters[(size_t)row * Hkv + kvh] = 0;
}

// A row with nothing visible (seq_len 0) gets zeros from its chunk-0 wavefront.
template <typename T>
__device__ void zero_heads(T* out, int row, int head0, int nh, int Hq, int D, int lane) {
  for (int h = 0; h < nh; ++h)
    for (int d = lane; d < D; d += 64) out[((size_t)row * Hq + head0 + h) * D + d] = from_f32<T>(0.f);
}

// ----------------------------------------------------------------------------
// fp16 pools, head_dim 128, MFMA scores.  G = query heads per KV head (1..8).
template <int G>
__global__ __launch_bounds__(64) void attn_chunk_f16_d128(
    const f16* __restrict__ q, const f16* __restrict__ kp, const f16* __restrict__ vp,
    const int32_t* __restrict__ pt, const int32_t* __restrict__ lens,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ counters, f16* __restrict__ out,
    int q_len, int Hq, int Hkv, int P, int max_pages, int NC, float scale_log2) {
  constexpr int D = 128;
  const int chunk = blockIdx.x, kvh = blockIdx.y, row = blockIdx.z;
  const int L = visible_len(lens, row, q_len, max_pages * P);
  const int t0 = chunk * kChunk;
  if (t0 >= L) {
    if (chunk == 0) zero_heads<f16>(out, row, kvh * G, G, Hq, D, threadIdx.x);
    return;
  }
  const int t1 = min(L, t0 + kChunk);
  const int b = row / q_len;
  const int lane = threadIdx.x;
  const int li = lane & 15;   // MFMA column (token within tile) / row of A
  const int lg = lane >> 4;   // k-group

  // Q as the A operand: row li = query head (kvh*G + li) if li < G; element e of
  // step s covers head dim 32*s + 8*lg + e (the same mapping K uses below).
  f16x8 qa[4];
  {
    const f16* qrow = q + ((size_t)row * Hq + (size_t)kvh * G + li) * D + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (li < G) {
        qa[s] = *reinterpret_cast<const f16x8*>(qrow + 32 * s);
      } else {
        qa[s] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
  }
  const int32_t* ptrow = pt + (size_t)b * max_pages;

  // Pass 1: scores.  sc[tile][r] = S[head 4*lg + r][token t0 + 16*tile + li].
  f32x4 sc[kTiles];
#pragma unroll
  for (int tile = 0; tile < kTiles; ++tile) {
    const int tt = t0 + 16 * tile;
    if (tt < t1) {
      const int page = ptrow[tt / P];
      const int off = tt - (tt / P) * P;
      const f16* krow = kp + (((size_t)page * Hkv + kvh) * P + off + li) * D + 8 * lg;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const f16x8 kb = *reinterpret_cast<const f16x8*>(krow + 32 * s);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[s], kb, acc, 0, 0, 0);
      }
      const bool valid = (tt + li) < t1;
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[tile][r] = valid ? acc[r] * scale_log2 : -INFINITY;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[tile][r] = -INFINITY;
    }
  }

  // Row max and sum per head (a row of 16 lanes shares the same 4 heads).
  float m[4], l[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float mx = -INFINITY;
#pragma unroll
    for (int tile = 0; tile < kTiles; ++tile) mx = fmaxf(mx, sc[tile][r]);
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    m[r] = mx;
    float sum = 0.f;
#pragma unroll
    for (int tile = 0; tile < kTiles; ++tile) {
      const float p = (sc[tile][r] == -INFINITY) ? 0.f : exp2f(sc[tile][r] - mx);
      sc[tile][r] = p;
      sum += p;
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
    l[r] = sum;
  }

  // Pass 2: O = P V.  Lane owns dims 8*li..8*li+7 of tokens 4*u + lg of each tile.
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

#pragma unroll
  for (int tile = 0; tile < kTiles; ++tile) {
    const int tt = t0 + 16 * tile;
    if (tt < t1) {
      const int page = ptrow[tt / P];
      const int off = tt - (tt / P) * P;
      const f16* vtile = vp + (((size_t)page * Hkv + kvh) * P + off) * D + 8 * li;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int tok = 4 * u + lg;
        const f16x8 vv = *reinterpret_cast<const f16x8*>(vtile + (size_t)tok * D);
        float vf[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = static_cast<float>(vv[e]);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          // p[h][tok] lives in lane tok + 16*(h/4), register h%4.
          const float p = __shfl(sc[tile][h & 3], tok + 16 * (h >> 2), 64);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(p, vf[e], acc[h][e]);
        }
      }
    }
  }
  // Sum the four token groups (lanes li, li+16, li+32, li+48).
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[h][e];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[h][e] = v;
    }

  if (lg == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const int head = kvh * G + h;
      float* dst = part_o + (((size_t)row * Hq + head) * NC + chunk) * D + 8 * li;
      *reinterpret_cast<float4*>(dst) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
    }
  }
  if (li == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int h = 4 * lg + r;
      if (h < G) {
        float* ml = part_ml + (((size_t)row * Hq + kvh * G + h) * NC + chunk) * 2;
        ml[0] = m[r];
        ml[1] = l[r];
      }
    }
  }
  finish_chunk<f16>(part_o, part_ml, counters, out, row, kvh, G, Hq, Hkv, D, NC, L, lane);
}

// ----------------------------------------------------------------------------
// Generic VALU kernel (fp32 or fp16 pools, any page size, head_dim <= 256).
template <typename T>
__global__ __launch_bounds__(64) void attn_chunk_generic(
    const T* __restrict__ q, const T* __restrict__ kp, const T* __restrict__ vp,
    const int32_t* __restrict__ pt, const int32_t* __restrict__ lens,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ counters, T* __restrict__ out,
    int q_len, int Hq, int Hkv, int D, int P, int max_pages, int NC, float scale_log2) {
  __shared__ float qs[256];
  __shared__ float ps[kChunk];
  const int chunk = blockIdx.x, kvh = blockIdx.y, row = blockIdx.z;
  const int L = visible_len(lens, row, q_len, max_pages * P);
  const int t0 = chunk * kChunk;
  const int G = Hq / Hkv;
  const int lane = threadIdx.x;
  if (t0 >= L) {
    if (chunk == 0) zero_heads<T>(out, row, kvh * G, G, Hq, D, lane);
    return;
  }
  const int n = min(L, t0 + kChunk) - t0;
  const int b = row / q_len;
  const int32_t* ptrow = pt + (size_t)b * max_pages;
  for (int h = 0; h < G; ++h) {
    const int head = kvh * G + h;
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
      float* ml = part_ml + (((size_t)row * Hq + head) * NC + chunk) * 2;
      ml[0] = mx;
      ml[1] = sum;
    }
  }
  finish_chunk<T>(part_o, part_ml, counters, out, row, kvh, G, Hq, Hkv, D, NC, L, lane);
}

int num_chunks(int max_context) { return max_context > 0 ? (max_context + kChunk - 1) / kChunk : 1; }

int launch_attention(const void* q, const void* k_pool, const void* v_pool, const int32_t* page_table,
                     const int32_t* seq_lens, void* out, void* workspace, size_t workspace_bytes,
                     int batch, int q_len, int Hq, int Hkv, int D, int P, int max_pages, float scale,
                     int kv_dtype, void* stream) {
  CIR_CHECK_ARG(batch >= 0 && q_len >= 1, "attention: batch must be >= 0 and q_len >= 1");
  if (batch == 0) return 0;
  CIR_CHECK_ARG(q && k_pool && v_pool && page_table && seq_lens && out && workspace, "attention: null pointer");
  CIR_CHECK_ARG(Hkv > 0 && Hq > 0 && Hq % Hkv == 0, "attention: num_heads (%d) must be a multiple of num_kv_heads (%d)", Hq, Hkv);
  CIR_CHECK_ARG(D > 0 && D <= 256, "attention: head_dim %d out of range (1..256)", D);
  CIR_CHECK_ARG(P > 0 && max_pages > 0, "attention: page_size and max_pages must be positive");
  CIR_CHECK_ARG(kv_dtype == CIR_F16 || kv_dtype == CIR_F32, "attention: kv_dtype must be CIR_F16 or CIR_F32");
  const int rows = batch * q_len;
  const int NC = num_chunks(max_pages * P);
  const size_t need = cir_paged_attention_workspace_bytes(rows, Hq, D, max_pages * P);
  CIR_CHECK_ARG(workspace_bytes >= need, "attention: workspace too small (%zu < %zu)", workspace_bytes, need);
  CIR_CHECK_ARG(rows <= 65535 && Hkv <= 65535, "attention: grid too large");
  float* part_o = static_cast<float*>(workspace);
  float* part_ml = part_o + (size_t)rows * Hq * NC * D;
  int* counters = reinterpret_cast<int*>(part_ml + (size_t)rows * Hq * NC * 2);
  const float scale_log2 = scale * kLog2e;
  const int G = Hq / Hkv;
  hipStream_t s = as_stream(stream);
  dim3 grid(NC, Hkv, rows);
  const bool mfma = kv_dtype == CIR_F16 && D == 128 && P % 16 == 0 && G <= 8;
  if (mfma) {
    auto kq = static_cast<const f16*>(q);
    auto kk = static_cast<const f16*>(k_pool);
    auto kv = static_cast<const f16*>(v_pool);
#define CIR_ATT_CASE(g)                                                                                    \
  case g:                                                                                                  \
    attn_chunk_f16_d128<g><<<grid, 64, 0, s>>>(kq, kk, kv, page_table, seq_lens, part_o, part_ml, counters,   \
                                               static_cast<f16*>(out), q_len, Hq, Hkv, P, max_pages, NC,  \
                                               scale_log2);                                                \
    break;
    switch (G) {
      CIR_ATT_CASE(1) CIR_ATT_CASE(2) CIR_ATT_CASE(3) CIR_ATT_CASE(4)
      CIR_ATT_CASE(5) CIR_ATT_CASE(6) CIR_ATT_CASE(7) CIR_ATT_CASE(8)
    }
#undef CIR_ATT_CASE
  } else if (kv_dtype == CIR_F16) {
    attn_chunk_generic<f16><<<grid, 64, 0, s>>>(static_cast<const f16*>(q), static_cast<const f16*>(k_pool),
                                                static_cast<const f16*>(v_pool), page_table, seq_lens, part_o,
                                                part_ml, counters, static_cast<f16*>(out), q_len, Hq, Hkv, D, P,
                                                max_pages, NC, scale_log2);
  } else {
    attn_chunk_generic<float><<<grid, 64, 0, s>>>(static_cast<const float*>(q), static_cast<const float*>(k_pool),
                                                  static_cast<const float*>(v_pool), page_table, seq_lens, part_o,
                                                  part_ml, counters, static_cast<float*>(out), q_len, Hq, Hkv, D, P,
                                                  max_pages, NC, scale_log2);
  }
  return launch_status();
}

}  // namespace
}  // namespace cir

extern "C" size_t cir_paged_attention_workspace_bytes(int rows, int num_heads, int head_dim, int max_context) {
  if (rows <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  const size_t nc = (size_t)cir::num_chunks(max_context);
  // partial O and (max, sum) per (row, head, chunk), then one ticket counter per (row, head)
  return (size_t)rows * num_heads * nc * ((size_t)head_dim + 2) * sizeof(float) + (size_t)rows * num_heads * sizeof(int);
}

extern "C" int cir_paged_decode_attention(const void* q, const void* k_pool, const void* v_pool,
                                          const int32_t* page_table, const int32_t* seq_lens, void* out,
                                          void* workspace, size_t workspace_bytes, int batch, int num_heads,
                                          int num_kv_heads, int head_dim, int page_size, int max_pages, float scale,
                                          int kv_dtype, void* stream) {
  return cir::launch_attention(q, k_pool, v_pool, page_table, seq_lens, out, workspace, workspace_bytes, batch, 1,
                               num_heads, num_kv_heads, head_dim, page_size, max_pages, scale, kv_dtype, stream);
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
