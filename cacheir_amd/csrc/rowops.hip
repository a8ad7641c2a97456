// Row-wise kernels around the GEMMs: embedding gather, RMSNorm, residual add,
// GEMM epilogues (split-k sum + residual / SwiGLU / RoPE + KV-page append) and
// greedy argmax.  Reference semantics are cited at each entry point in
// include/cacheir_hip.h.
#include "common.hpp"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>

namespace cir {

static thread_local char g_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

namespace {

bool valid_dt(int dt) { return dt == CIR_F32 || dt == CIR_F16; }

// ---------------------------------------------------------------- rmsnorm ----
constexpr int kRowThreads = 1024;
constexpr int kRowVals = 8;  // rows up to 8192 stay in registers

// Block-wide sum over 1024 threads (16 wavefronts).
__device__ __forceinline__ float block_sum_1024(float v, float* scratch) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kRowThreads / 64; ++w) t += scratch[w];
  return t;
}

template <typename TX, typename TW, typename TO>
__global__ __launch_bounds__(kRowThreads) void rmsnorm_kernel(const TX* __restrict__ x, const TW* __restrict__ w,
                                                              TO* __restrict__ out, int hidden, float eps) {
  __shared__ float scratch[kRowThreads / 64];
  const int r = blockIdx.x;
  const TX* xr = x + (size_t)r * hidden;
  float v[kRowVals];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kRowVals; ++i) {
    const int c = threadIdx.x + i * kRowThreads;
    v[i] = c < hidden ? to_f32(xr[c]) : 0.f;
    ss = fmaf(v[i], v[i], ss);
  }
  for (int c = threadIdx.x + kRowVals * kRowThreads; c < hidden; c += kRowThreads) {
    const float t = to_f32(xr[c]);
    ss = fmaf(t, t, ss);
  }
  const float scale = 1.0f / sqrtf(block_sum_1024(ss, scratch) / (float)hidden + eps);
  TO* o = out + (size_t)r * hidden;
#pragma unroll
  for (int i = 0; i < kRowVals; ++i) {
    const int c = threadIdx.x + i * kRowThreads;
    if (c < hidden) o[c] = from_f32<TO>((v[i] * scale) * to_f32(w[c]));
  }
  for (int c = threadIdx.x + kRowVals * kRowThreads; c < hidden; c += kRowThreads)
    o[c] = from_f32<TO>((to_f32(xr[c]) * scale) * to_f32(w[c]));
}

// Sum of `splits` (<= SMAX) partial planes at idx; every load is issued before the
// adds (indices past `splits` re-read plane 0 and are dropped), in fixed order.
template <int SMAX>
__device__ __forceinline__ float4 split_sum4(const float* __restrict__ part, int splits, size_t plane, size_t idx) {
  float4 v[SMAX];
#pragma unroll
  for (int sp = 0; sp < SMAX; ++sp) v[sp] = *reinterpret_cast<const float4*>(part + (sp < splits ? sp : 0) * plane + idx);
  float4 t = v[0];
#pragma unroll
  for (int sp = 1; sp < SMAX; ++sp)
    if (sp < splits) {
      t.x += v[sp].x;
      t.y += v[sp].y;
      t.z += v[sp].z;
      t.w += v[sp].w;
    }
  return t;
}

// Four consecutive values as one vector access (8 B for fp16, 16 B for fp32).
__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load4(const f16* p) {
  const f16x4 h = *reinterpret_cast<const f16x4*>(p);
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}
__device__ __forceinline__ void store4(float* p, float4 v) { *reinterpret_cast<float4*>(p) = v; }
__device__ __forceinline__ void store4(f16* p, float4 v) {
  *reinterpret_cast<f16x4*>(p) = f16x4{(f16)v.x, (f16)v.y, (f16)v.z, (f16)v.w};
}

// ---------------------------------------------------------------- embedding --
// One workgroup per row.  VEC: hidden % 4 == 0 and 16-byte aligned rows, 4 values per
// access with kEmbUnroll accesses of a thread issued before its first store (a row of
// 4096 is one round trip); otherwise one value at a time.
constexpr int kEmbThreads = 256;
constexpr int kEmbUnroll = 4;
template <typename TT, typename TO, bool VEC>
__global__ __launch_bounds__(kEmbThreads) void embedding_kernel(const int64_t* __restrict__ ids,
                                                                const TT* __restrict__ table, TO* __restrict__ out,
                                                                int hidden, int vocab) {
  const int r = blockIdx.x;
  int64_t id = ids[r];
  // Out-of-range ids are clamped, so no id reads outside the table; the runtime
  // rejects them on the host before they get here.
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  const TT* src = table + (size_t)id * hidden;
  TO* dst = out + (size_t)r * hidden;
  if constexpr (VEC) {
    const int n4 = hidden / 4;
    for (int base = threadIdx.x; base < n4; base += kEmbThreads * kEmbUnroll) {
      float4 v[kEmbUnroll];
#pragma unroll
      for (int u = 0; u < kEmbUnroll; ++u) {
        const int i = base + u * kEmbThreads;
        if (i < n4) v[u] = load4(src + 4 * i);
      }
#pragma unroll
      for (int u = 0; u < kEmbUnroll; ++u) {
        const int i = base + u * kEmbThreads;
        if (i < n4) store4(dst + 4 * i, v[u]);
      }
    }
  } else {
    for (int i = threadIdx.x; i < hidden; i += kEmbThreads) dst[i] = from_f32<TO>(to_f32(src[i]));
  }
}

// Residual epilogue + RMSNorm of the result, one workgroup per row, 4 columns per
// thread per step: h = residual + sum of partials (fp32, to h_out) and
// xn = (h * rsqrt(mean(h^2) + eps)) * w.  N % 4 == 0 and N <= 8192; TWO (N > 4096)
// gives each thread a second column group.  Every load of a column group (its partials,
// the residual, the norm weights) is issued before the group's first add, so a row costs
// one memory round trip; with more than 8 splits the two groups of a TWO row are loaded
// and summed one after the other (two round trips): both groups' 16 float4 partials at
// once would take 128 VGPRs and spill.
template <int SMAX, bool TWO, typename TW, typename TO>
__global__ __launch_bounds__(kRowThreads) void residual_rmsnorm_kernel(
    const float* __restrict__ part, int splits, const float* __restrict__ resid, float* __restrict__ h_out,
    const TW* __restrict__ w, TO* __restrict__ xn, int M, int N, float eps) {
  __shared__ float scratch[kRowThreads / 64];
  const int r = blockIdx.x;
  const size_t plane = (size_t)M * N;
  constexpr int G = TWO ? 2 : 1;
  constexpr bool kSeq = TWO && SMAX > 8;
  float4 v[G], wv[G];
  size_t idx[G];
  bool ok[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int c = 4 * (threadIdx.x + i * kRowThreads);
    ok[i] = c < N;
    idx[i] = (size_t)r * N + (ok[i] ? c : 0);
  }
  auto load = [&](int i, float4 (&pv)[SMAX], float4& q) __attribute__((always_inline)) {
#pragma unroll
    for (int sp = 0; sp < SMAX; ++sp)
      pv[sp] = *reinterpret_cast<const float4*>(part + (sp < splits ? sp : 0) * plane + idx[i]);
    q = *reinterpret_cast<const float4*>(resid + idx[i]);
    wv[i] = load4(w + (idx[i] - (size_t)r * N));
  };
  float ss = 0.f;
  // partials in split order, then the residual (as split_sum4 + add)
  auto fold = [&](int i, const float4 (&pv)[SMAX], const float4& q) __attribute__((always_inline)) {
    float4 t = {0.f, 0.f, 0.f, 0.f};
    if (ok[i]) {
      float4 p = pv[0];
#pragma unroll
      for (int sp = 1; sp < SMAX; ++sp)
        if (sp < splits) {
          p.x += pv[sp].x;
          p.y += pv[sp].y;
          p.z += pv[sp].z;
          p.w += pv[sp].w;
        }
      t = make_float4(q.x + p.x, q.y + p.y, q.z + p.z, q.w + p.w);
      *reinterpret_cast<float4*>(h_out + idx[i]) = t;
    }
    v[i] = t;
    ss += t.x * t.x + t.y * t.y + t.z * t.z + t.w * t.w;
  };
  if constexpr (kSeq) {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      float4 pv[SMAX], q;
      load(i, pv, q);
      fold(i, pv, q);
      __builtin_amdgcn_sched_barrier(0);  // the next group's loads stay behind these sums
    }
  } else {
    float4 pv[G][SMAX], q[G];
#pragma unroll
    for (int i = 0; i < G; ++i) load(i, pv[i], q[i]);
#pragma unroll
    for (int i = 0; i < G; ++i) fold(i, pv[i], q[i]);
  }
  const float scale = 1.0f / sqrtf(block_sum_1024(ss, scratch) / (float)N + eps);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    if (ok[i])
      store4(xn + idx[i], make_float4((v[i].x * scale) * wv[i].x, (v[i].y * scale) * wv[i].y,
                                      (v[i].z * scale) * wv[i].z, (v[i].w * scale) * wv[i].w));
  }
}

template <typename T>
__global__ void add_kernel(const T* __restrict__ a, const T* __restrict__ b, T* __restrict__ out, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = from_f32<T>(to_f32(a[i]) + to_f32(b[i]));
}

template <typename TI, typename TO>
__global__ void cast_kernel(const TI* __restrict__ in, TO* __restrict__ out, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = from_f32<TO>(to_f32(in[i]));
}

// ---------------------------------------------------------------- epilogues --
// out = (residual +) sum of partials, 4 elements per thread (M*N % 4 == 0).
template <int SMAX, typename T>
__global__ void epi_store_kernel(const float* __restrict__ part, int splits, const T* __restrict__ resid,
                                 T* __restrict__ out, int M, int N) {
  const size_t n_el = (size_t)M * N;
  const size_t i = 4 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n_el) return;
  float4 v = split_sum4<SMAX>(part, splits, n_el, i);
  if (resid) {
    v.x += to_f32(resid[i]);
    v.y += to_f32(resid[i + 1]);
    v.z += to_f32(resid[i + 2]);
    v.w += to_f32(resid[i + 3]);
  }
  out[i] = from_f32<T>(v.x);
  out[i + 1] = from_f32<T>(v.y);
  out[i + 2] = from_f32<T>(v.z);
  out[i + 3] = from_f32<T>(v.w);
}

__device__ __forceinline__ float silu_mul1(float g, float u) { return as_f32_value((g / (1.0f + expf(-g))) * u); }

// SwiGLU over [gate | up] partial columns, 4 outputs per thread (I % 4 == 0).
template <int SMAX, typename T>
__global__ void epi_swiglu_kernel(const float* __restrict__ part, int splits, T* __restrict__ out, int M, int I) {
  const size_t n_el = (size_t)M * I;
  const size_t i = 4 * ((size_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (i >= n_el) return;
  const int m = (int)(i / I), j = (int)(i % I);
  const size_t plane = (size_t)M * 2 * I;
  const float4 g = split_sum4<SMAX>(part, splits, plane, (size_t)m * 2 * I + j);
  const float4 u = split_sum4<SMAX>(part, splits, plane, (size_t)m * 2 * I + I + j);
  out[i] = from_f32<T>(silu_mul1(g.x, u.x));
  out[i + 1] = from_f32<T>(silu_mul1(g.y, u.y));
  out[i + 2] = from_f32<T>(silu_mul1(g.z, u.z));
  out[i + 3] = from_f32<T>(silu_mul1(g.w, u.w));
}

// Sum of `splits` partial planes for the two columns idx, idx + 1 (idx even), added in split order as split_sum.
__device__ __forceinline__ float2 split_sum2(const float* __restrict__ part, int splits, size_t plane, size_t idx) {
  float2 v = *reinterpret_cast<const float2*>(part + idx);
  for (int s = 1; s < splits; ++s) {
    const float2 t = *reinterpret_cast<const float2*>(part + (size_t)s * plane + idx);
    v.x += t.x;
    v.y += t.y;
  }
  return v;
}

// Heads whose rotation pair i one thread rotates with one sincosf: at prompt positions in the thousands the
// argument pos * inv_freq[i] takes the long range reduction, which cost more than the epilogue's memory traffic
// when every (head, pair) evaluated it.
constexpr int kRopeHeads = 8;

// Columns: q [Hq*D], k [Hkv*D], v [Hkv*D], so q head h and k head h - Hq both start at column h*D.  Per row, one
// thread per (group of kRopeHeads q/k heads, rotation pair i), then one per (v head, column pair).
template <typename TQ, typename TK>
__global__ void epi_qkv_kernel(const float* __restrict__ part, int splits, const float* __restrict__ inv_freq,
                               const int32_t* __restrict__ positions, const int32_t* __restrict__ pt, int max_pages,
                               TQ* __restrict__ q_out, TK* __restrict__ kp, TK* __restrict__ vp, int q_len, int Hq,
                               int Hkv, int D, int P, int rows) {
  const int half = D / 2;
  const int H = Hq + Hkv;
  const int rot = (H + kRopeHeads - 1) / kRopeHeads * half;
  const int per_row = rot + Hkv * half;
  // 32-bit unsigned index arithmetic (the launcher keeps rows * per_row below 2^31)
  const unsigned id = blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (unsigned)(rows * per_row)) return;
  const int r = (int)(id / (unsigned)per_row);
  const int c = (int)(id % (unsigned)per_row);
  const int b = (int)((unsigned)r / (unsigned)q_len), s = r - b * q_len;
  const int pos = positions[b] + s;
  const size_t plane = (size_t)rows * (H + Hkv) * D;
  const float* base = part + (size_t)r * (H + Hkv) * D;
  const int page_idx = pos / P;
  const int slot = (page_idx < max_pages) ? pt[(size_t)b * max_pages + page_idx] : -1;
  const int off = pos - page_idx * P;
  if (c < rot) {
    const int hq = (int)((unsigned)c / (unsigned)half), i = c - hq * half, h0 = hq * kRopeHeads;
    float sn, cs;
    sincosf((float)pos * inv_freq[i], &sn, &cs);
#pragma unroll
    for (int u = 0; u < kRopeHeads; ++u) {
      const int h = h0 + u;
      if (h >= H) break;
      const float2 x = split_sum2(base, splits, plane, (size_t)h * D + 2 * i);
      // The fused decode attention prologue rotates the same values with these same operations: each FMA written
      // out (not left to contraction) and rounded to fp32 before an fp16 store (no single-rounding mixed FMA).
      const float y0 = as_f32_value(fmaf(x.x, cs, -(x.y * sn)));
      const float y1 = as_f32_value(fmaf(x.x, sn, x.y * cs));
      if (h < Hq) {
        TQ* o = q_out + ((size_t)r * Hq + h) * D + 2 * i;
        o[0] = from_f32<TQ>(y0);
        o[1] = from_f32<TQ>(y1);
      } else if (slot >= 0) {
        TK* o = kp + (((size_t)slot * Hkv + (h - Hq)) * P + off) * D + 2 * i;
        o[0] = from_f32<TK>(y0);
        o[1] = from_f32<TK>(y1);
      }
    }
  } else if (slot >= 0) {
    const int cc = c - rot;
    const int head = (int)((unsigned)cc / (unsigned)half), d = 2 * (cc - head * half);
    const float2 v = split_sum2(base, splits, plane, (size_t)(H + head) * D + d);
    TK* o = vp + (((size_t)slot * Hkv + head) * P + off) * D + d;
    o[0] = from_f32<TK>(v.x);
    o[1] = from_f32<TK>(v.y);
  }
}

// ---------------------------------------------------------------- argmax -----
__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) { argmax_better(bv, bi, v, i); }

__global__ __launch_bounds__(kRowThreads) void argmax_kernel(const float* __restrict__ logits, int ld,
                                                             int64_t* __restrict__ ids, int vocab) {
  __shared__ float sv[kRowThreads / 64];
  __shared__ int si[kRowThreads / 64];
  const int r = blockIdx.x;
  const float* row = logits + (size_t)r * ld;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  constexpr int U = 4;
  int base = threadIdx.x;
  for (; base + (U - 1) * kRowThreads < vocab; base += U * kRowThreads) {
    float t[U];
#pragma unroll
    for (int u = 0; u < U; ++u) t[u] = row[base + u * kRowThreads];
#pragma unroll
    for (int u = 0; u < U; ++u) better(bv, bi, t[u], base + u * kRowThreads);
  }
  for (int i = base; i < vocab; i += kRowThreads) better(bv, bi, row[i], i);
  // wavefront then workgroup reduction, ties to the smaller index
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    better(bv, bi, ov, oi);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kRowThreads / 64; ++w) better(bv, bi, sv[w], si[w]);
    ids[r] = bi == 0x7fffffff ? 0 : bi;
  }
}

unsigned blocks_for(size_t n, unsigned bs) { return (unsigned)((n + bs - 1) / bs); }

// Calls f.template operator()<SMAX>() with the smallest SMAX in {1, 2, 4, 8, 16} >= splits.
template <typename F>
int with_smax(int splits, F&& f) {
  if (splits <= 1) return f.template operator()<1>();
  if (splits <= 2) return f.template operator()<2>();
  if (splits <= 4) return f.template operator()<4>();
  if (splits <= 8) return f.template operator()<8>();
  if (splits <= 16) return f.template operator()<16>();
  set_error("epilogue: at most 16 k-splits (got %d)", splits);
  return static_cast<int>(hipErrorInvalidValue);
}

}  // namespace
}  // namespace cir

using namespace cir;

extern "C" const char* cir_version(void) { return "cacheir_amd 0.1 gfx950"; }
extern "C" const char* cir_last_error_string(void) { return cir::g_error; }

extern "C" int cir_embedding(const int64_t* ids, const void* table, int tdt, void* out, int odt, int rows, int hidden,
                             int vocab, void* stream) {
  CIR_CHECK_ARG(valid_dt(tdt) && valid_dt(odt), "embedding: bad dtype");
  CIR_CHECK_ARG(rows >= 0 && hidden >= 0 && vocab > 0, "embedding: bad sizes");
  if (rows == 0 || hidden == 0) return 0;
  CIR_CHECK_ARG(ids && table && out, "embedding: null pointer");
  hipStream_t s = as_stream(stream);
  // 4-value accesses need every row 8- (fp16) or 16-byte (fp32) aligned: base pointers on 16 bytes, hidden % 4 == 0.
  const bool vec = hidden % 4 == 0 && reinterpret_cast<uintptr_t>(table) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(out) % 16 == 0;
  auto go = [&]<typename TT, typename TO>() {
    if (vec) embedding_kernel<TT, TO, true><<<rows, kEmbThreads, 0, s>>>(ids, (const TT*)table, (TO*)out, hidden, vocab);
    else embedding_kernel<TT, TO, false><<<rows, kEmbThreads, 0, s>>>(ids, (const TT*)table, (TO*)out, hidden, vocab);
  };
  if (tdt == CIR_F32 && odt == CIR_F32) go.template operator()<float, float>();
  else if (tdt == CIR_F16 && odt == CIR_F32) go.template operator()<f16, float>();
  else if (tdt == CIR_F16 && odt == CIR_F16) go.template operator()<f16, f16>();
  else go.template operator()<float, f16>();
  return launch_status();
}

extern "C" int cir_rmsnorm(const void* x, int xdt, const void* w, int wdt, void* out, int odt, int rows, int hidden,
                           float eps, void* stream) {
  CIR_CHECK_ARG(valid_dt(xdt) && valid_dt(wdt) && valid_dt(odt), "rmsnorm: bad dtype");
  CIR_CHECK_ARG(rows >= 0 && hidden >= 0, "rmsnorm: bad sizes");
  if (rows == 0 || hidden == 0) return 0;
  CIR_CHECK_ARG(x && w && out, "rmsnorm: null pointer");
  hipStream_t s = as_stream(stream);
#define CIR_RMS(TX, TW, TO) \
  rmsnorm_kernel<TX, TW, TO><<<rows, kRowThreads, 0, s>>>((const TX*)x, (const TW*)w, (TO*)out, hidden, eps)
  const int key = xdt * 4 + wdt * 2 + odt;
  switch (key) {
    case 0: CIR_RMS(float, float, float); break;
    case 1: CIR_RMS(float, float, f16); break;
    case 2: CIR_RMS(float, f16, float); break;
    case 3: CIR_RMS(float, f16, f16); break;
    case 4: CIR_RMS(f16, float, float); break;
    case 5: CIR_RMS(f16, float, f16); break;
    case 6: CIR_RMS(f16, f16, float); break;
    default: CIR_RMS(f16, f16, f16); break;
  }
#undef CIR_RMS
  return launch_status();
}

extern "C" int cir_add(const void* a, const void* b, void* out, int dt, size_t count, void* stream) {
  CIR_CHECK_ARG(valid_dt(dt), "add: bad dtype");
  if (count == 0) return 0;
  CIR_CHECK_ARG(a && b && out, "add: null pointer");
  hipStream_t s = as_stream(stream);
  if (dt == CIR_F32)
    add_kernel<float><<<blocks_for(count, 256), 256, 0, s>>>((const float*)a, (const float*)b, (float*)out, count);
  else
    add_kernel<f16><<<blocks_for(count, 256), 256, 0, s>>>((const f16*)a, (const f16*)b, (f16*)out, count);
  return launch_status();
}

extern "C" int cir_cast(const void* in, int idt, void* out, int odt, size_t count, void* stream) {
  CIR_CHECK_ARG(valid_dt(idt) && valid_dt(odt), "cast: bad dtype");
  if (count == 0) return 0;
  CIR_CHECK_ARG(in && out, "cast: null pointer");
  hipStream_t s = as_stream(stream);
  const unsigned nb = blocks_for(count, 256);
  if (idt == CIR_F32 && odt == CIR_F16) cast_kernel<float, f16><<<nb, 256, 0, s>>>((const float*)in, (f16*)out, count);
  else if (idt == CIR_F16 && odt == CIR_F32) cast_kernel<f16, float><<<nb, 256, 0, s>>>((const f16*)in, (float*)out, count);
  else if (idt == CIR_F32) cast_kernel<float, float><<<nb, 256, 0, s>>>((const float*)in, (float*)out, count);
  else cast_kernel<f16, f16><<<nb, 256, 0, s>>>((const f16*)in, (f16*)out, count);
  return launch_status();
}

extern "C" int cir_epilogue_store(const float* y_partial, int splits, const void* residual, void* out, int odt, int m,
                                  int n, void* stream) {
  CIR_CHECK_ARG(valid_dt(odt) && splits >= 1 && m >= 0 && n >= 0, "epilogue_store: bad arguments");
  if (m == 0 || n == 0) return 0;
  CIR_CHECK_ARG(((size_t)m * n) % 4 == 0, "epilogue_store: m*n must be a multiple of 4");
  CIR_CHECK_ARG(y_partial && out, "epilogue_store: null pointer");
  hipStream_t s = as_stream(stream);
  const unsigned nb = blocks_for((size_t)m * n / 4, 256);
  return with_smax(splits, [&]<int S>() {
    if (odt == CIR_F32)
      epi_store_kernel<S, float><<<nb, 256, 0, s>>>(y_partial, splits, (const float*)residual, (float*)out, m, n);
    else
      epi_store_kernel<S, f16><<<nb, 256, 0, s>>>(y_partial, splits, (const f16*)residual, (f16*)out, m, n);
    return launch_status();
  });
}

extern "C" int cir_epilogue_residual_rmsnorm(const float* y_partial, int splits, const float* residual, float* h_out,
                                             const void* norm_w, int wdt, float eps, void* xn, int xdt, int m, int n,
                                             void* stream) {
  CIR_CHECK_ARG(valid_dt(wdt) && valid_dt(xdt) && splits >= 1 && m >= 0 && n >= 0, "epilogue_residual_rmsnorm: bad arguments");
  if (m == 0 || n == 0) return 0;
  CIR_CHECK_ARG(n % 4 == 0 && n <= 8 * kRowThreads, "epilogue_residual_rmsnorm: row length %d must be a multiple of 4 and <= %d",
                n, 8 * kRowThreads);
  CIR_CHECK_ARG(y_partial && residual && h_out && norm_w && xn, "epilogue_residual_rmsnorm: null pointer");
  hipStream_t s = as_stream(stream);
  return with_smax(splits, [&]<int S>() {
#define CIR_RR(TW, TO)                                                                                           \
  do {                                                                                                           \
    if (n > 4 * kRowThreads)                                                                                     \
      residual_rmsnorm_kernel<S, true, TW, TO><<<m, kRowThreads, 0, s>>>(y_partial, splits, residual, h_out,     \
                                                                         (const TW*)norm_w, (TO*)xn, m, n, eps); \
    else                                                                                                         \
      residual_rmsnorm_kernel<S, false, TW, TO><<<m, kRowThreads, 0, s>>>(y_partial, splits, residual, h_out,    \
                                                                          (const TW*)norm_w, (TO*)xn, m, n, eps); \
  } while (0)
    if (wdt == CIR_F32 && xdt == CIR_F32) CIR_RR(float, float);
    else if (wdt == CIR_F32 && xdt == CIR_F16) CIR_RR(float, f16);
    else if (wdt == CIR_F16 && xdt == CIR_F32) CIR_RR(f16, float);
    else CIR_RR(f16, f16);
#undef CIR_RR
    return launch_status();
  });
}

extern "C" int cir_epilogue_swiglu(const float* y_partial, int splits, void* out, int odt, int m, int inter, void* stream) {
  CIR_CHECK_ARG(valid_dt(odt) && splits >= 1 && m >= 0 && inter >= 0, "epilogue_swiglu: bad arguments");
  if (m == 0 || inter == 0) return 0;
  CIR_CHECK_ARG(inter % 4 == 0, "epilogue_swiglu: intermediate size must be a multiple of 4");
  CIR_CHECK_ARG(y_partial && out, "epilogue_swiglu: null pointer");
  hipStream_t s = as_stream(stream);
  const unsigned nb = blocks_for((size_t)m * inter / 4, 256);
  return with_smax(splits, [&]<int S>() {
    if (odt == CIR_F32)
      epi_swiglu_kernel<S, float><<<nb, 256, 0, s>>>(y_partial, splits, (float*)out, m, inter);
    else
      epi_swiglu_kernel<S, f16><<<nb, 256, 0, s>>>(y_partial, splits, (f16*)out, m, inter);
    return launch_status();
  });
}

extern "C" int cir_epilogue_qkv_rope_append(const float* y_partial, int splits, const float* inv_freq,
                                            const int32_t* positions, const int32_t* page_table, int max_pages,
                                            void* q_out, int odt, void* k_pool, void* v_pool, int kvt, int batch,
                                            int q_len, int num_heads, int num_kv_heads, int head_dim, int page_size,
                                            void* stream) {
  CIR_CHECK_ARG(valid_dt(odt) && valid_dt(kvt) && splits >= 1, "epilogue_qkv: bad dtype/splits");
  CIR_CHECK_ARG(batch >= 0 && q_len >= 1 && head_dim > 0 && head_dim % 2 == 0 && num_heads > 0 && num_kv_heads > 0 &&
                    page_size > 0 && max_pages > 0,
                "epilogue_qkv: bad sizes");
  if (batch == 0) return 0;
  CIR_CHECK_ARG(y_partial && inv_freq && positions && page_table && q_out && k_pool && v_pool, "epilogue_qkv: null pointer");
  const int rows = batch * q_len;
  const int rope_groups = (num_heads + num_kv_heads + kRopeHeads - 1) / kRopeHeads;
  const long total = (long)rows * (rope_groups + num_kv_heads) * (head_dim / 2);
  CIR_CHECK_ARG(total < (1L << 31), "epilogue_qkv: %ld work items exceed the kernel's 32-bit index", total);
  hipStream_t s = as_stream(stream);
  const unsigned nb = (unsigned)((total + 255) / 256);
#define CIR_QKV(TQ, TK)                                                                                            \
  epi_qkv_kernel<TQ, TK><<<nb, 256, 0, s>>>(y_partial, splits, inv_freq, positions, page_table, max_pages, (TQ*)q_out, \
                                            (TK*)k_pool, (TK*)v_pool, q_len, num_heads, num_kv_heads, head_dim,      \
                                            page_size, rows)
  if (odt == CIR_F32 && kvt == CIR_F32) CIR_QKV(float, float);
  else if (odt == CIR_F16 && kvt == CIR_F16) CIR_QKV(f16, f16);
  else if (odt == CIR_F32 && kvt == CIR_F16) CIR_QKV(float, f16);
  else CIR_QKV(f16, float);
#undef CIR_QKV
  return launch_status();
}

extern "C" int cir_argmax(const float* logits, int ld, int64_t* ids, int rows, int vocab, void* stream) {
  CIR_CHECK_ARG(rows >= 0 && vocab > 0 && ld >= vocab, "argmax: bad sizes");
  if (rows == 0) return 0;
  CIR_CHECK_ARG(logits && ids, "argmax: null pointer");
  argmax_kernel<<<rows, kRowThreads, 0, as_stream(stream)>>>(logits, ld, ids, vocab);
  return launch_status();
}
