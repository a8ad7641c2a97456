/*
 * C/OpenMP restatement of the CacheIR CPU decode-step arithmetic -- TEST
 * INFRASTRUCTURE ONLY (timed CPU baseline in bench.py; never on the product path).
 *
 * Semantics follow the reference CPU runtime (cacheir/runtime/cpu.py:221-377) with
 * GGUF Q4_0 weights decoded as gguf.py:297-310 does, but on the fly per block
 * instead of once into fp32 (the arithmetic per weight is the same exact
 * (nib - 8) * d in fp32).  The reference's own native CPU kernels
 * (cpp/src/cacheir_backend.cpp:91-165: rms_norm, silu_mul, out x in matmul with an
 * OpenMP row loop) are the model for the structure: OpenMP over output rows / over
 * (sequence, KV head), fp32 accumulation, vectorisable inner loops.
 *
 * Built by oracle/Makefile into oracle/_lib/liboracle_cpu.so.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <string.h>

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

int orc_threads(void) { return omp_get_max_threads(); }

/* cpu.py:284-289 */
void orc_rmsnorm(const float* x, const float* w, float* out, int rows, int hidden, float eps) {
#pragma omp parallel for
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * hidden;
    float ss = 0.f;
    for (int i = 0; i < hidden; ++i) ss += xr[i] * xr[i];
    const float scale = 1.0f / sqrtf(ss / (float)hidden + eps);
    for (int i = 0; i < hidden; ++i) out[(size_t)r * hidden + i] = (xr[i] * scale) * w[i];
  }
}

/* 16 fp16 values -> fp32 (F16C / AVX-512 conversions). */
static inline void h2f16(const uint16_t* src, float* dst) {
#ifdef __AVX512F__
  _mm512_storeu_ps(dst, _mm512_cvtph_ps(_mm256_loadu_si256((const __m256i*)src)));
#else
  _mm256_storeu_ps(dst, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)src)));
  _mm256_storeu_ps(dst + 8, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(src + 8))));
#endif
}

/* y[m][n] (+)= sum_k x[m][k] * W[n][k] with W in GGUF Q4_0 blocks (18 bytes / 32 values);
 * accumulate != 0 adds into y (the residual add of cpu.py:256-257). M <= 64.
 * Each row keeps 16 lane sums (lane j adds columns 32b + j and 32b + 16 + j of every
 * block b, in block order) reduced once at the end, so the inner loop is a plain
 * 16-wide vector FMA without reassociating any sum. */
void orc_q4_0_gemm(const float* x, int M, int K, const uint8_t* blocks, int N, float* y, int accumulate) {
  const int nb = K / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    float acc[64][16];
    for (int m = 0; m < M; ++m)
      for (int j = 0; j < 16; ++j) acc[m][j] = 0.f;
    const uint8_t* row = blocks + (size_t)n * nb * 18;
    for (int b = 0; b < nb; ++b) {
      const uint8_t* blk = row + (size_t)b * 18;
      const float d = h2f((uint16_t)(blk[0] | (blk[1] << 8)));
      float lo[16], hi[16];
      for (int j = 0; j < 16; ++j) {
        lo[j] = (float)((int)(blk[2 + j] & 15) - 8) * d;
        hi[j] = (float)((int)(blk[2 + j] >> 4) - 8) * d;
      }
      for (int m = 0; m < M; ++m) {
        const float* xm = x + (size_t)m * K + (size_t)b * 32;
        for (int j = 0; j < 16; ++j) acc[m][j] += lo[j] * xm[j] + hi[j] * xm[j + 16];
      }
    }
    for (int m = 0; m < M; ++m) {
      float s = 0.f;
      for (int j = 0; j < 16; ++j) s += acc[m][j];
      if (accumulate) y[(size_t)m * N + n] += s;
      else y[(size_t)m * N + n] = s;
    }
  }
}

/* Interleaved RoPE (cpu.py:324-340) on rows [rows][heads*D] at positions pos[r]. */
void orc_rope(float* x, int rows, int heads, int D, const int* pos, const float* inv_freq) {
#pragma omp parallel for
  for (int r = 0; r < rows; ++r) {
    for (int h = 0; h < heads; ++h) {
      float* v = x + ((size_t)r * heads + h) * D;
      for (int i = 0; i < D / 2; ++i) {
        const float a = (float)pos[r] * inv_freq[i];
        const float c = cosf(a), s = sinf(a);
        const float e = v[2 * i], o = v[2 * i + 1];
        v[2 * i] = e * c - o * s;
        v[2 * i + 1] = e * s + o * c;
      }
    }
  }
}

/* Append one token per sequence into fp16 pools [slots][Hkv][P][D] (kv_cache.py:66-79 as pages). */
void orc_kv_append(const float* k, const float* v, uint16_t* kp, uint16_t* vp, const int* page_table, int max_pages,
                   const int* pos, int B, int Hkv, int D, int P) {
  for (int b = 0; b < B; ++b) {
    const int slot = page_table[(size_t)b * max_pages + pos[b] / P], off = pos[b] % P;
    for (int h = 0; h < Hkv; ++h)
      for (int d = 0; d < D; ++d) {
        const size_t dst = (((size_t)slot * Hkv + h) * P + off) * D + d;
        kp[dst] = _cvtss_sh(k[((size_t)b * Hkv + h) * D + d], 0);
        vp[dst] = _cvtss_sh(v[((size_t)b * Hkv + h) * D + d], 0);
      }
  }
}

/* Paged decode attention over fp16 pools (cpu.py:342-377 semantics, GQA kvh = h / G). */
void orc_paged_attention(const float* q, const uint16_t* kp, const uint16_t* vp, const int* page_table, int max_pages,
                         const int* lens, float* out, int B, int Hq, int Hkv, int D, int P, float scale,
                         float* scratch /* [threads][max_ctx] */, int max_ctx) {
  const int G = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int b = 0; b < B; ++b) {
    for (int g = 0; g < Hkv; ++g) {
      float* sc = scratch + (size_t)omp_get_thread_num() * max_ctx;
      const int L = lens[b];
      for (int hh = 0; hh < G; ++hh) {
        const int h = g * G + hh;
        const float* qh = q + ((size_t)b * Hq + h) * D;
        float mx = -INFINITY;
        for (int t = 0; t < L; ++t) {
          const uint16_t* kr = kp + (((size_t)page_table[(size_t)b * max_pages + t / P] * Hkv + g) * P + t % P) * D;
          float part[16] = {0.f}, kf[16];
          int d = 0;
          for (; d + 16 <= D; d += 16) {
            h2f16(kr + d, kf);
            for (int j = 0; j < 16; ++j) part[j] += qh[d + j] * kf[j];
          }
          float s = 0.f;
          for (int j = 0; j < 16; ++j) s += part[j];
          for (; d < D; ++d) s += qh[d] * h2f(kr[d]);
          sc[t] = s * scale;
          if (sc[t] > mx) mx = sc[t];
        }
        float sum = 0.f;
        for (int t = 0; t < L; ++t) {
          sc[t] = expf(sc[t] - mx);
          sum += sc[t];
        }
        float* o = out + ((size_t)b * Hq + h) * D;
        for (int d = 0; d < D; ++d) o[d] = 0.f;
        for (int t = 0; t < L; ++t) {
          const uint16_t* vr = vp + (((size_t)page_table[(size_t)b * max_pages + t / P] * Hkv + g) * P + t % P) * D;
          const float p = sc[t] / sum;
          float vf[16];
          int d = 0;
          for (; d + 16 <= D; d += 16) {
            h2f16(vr + d, vf);
            for (int j = 0; j < 16; ++j) o[d + j] += p * vf[j];
          }
          for (; d < D; ++d) o[d] += p * h2f(vr[d]);
        }
      }
    }
  }
}

/* silu(g) * u (cpu.py:266-279); gu is [rows][2*I] = gate | up. */
void orc_silu_mul(const float* gu, float* out, int rows, int I) {
#pragma omp parallel for
  for (int r = 0; r < rows; ++r)
    for (int j = 0; j < I; ++j) {
      const float g = gu[(size_t)r * 2 * I + j], u = gu[(size_t)r * 2 * I + I + j];
      out[(size_t)r * I + j] = (g / (1.0f + expf(-g))) * u;
    }
}

/* First-index argmax per row (cpu.py:181-182). */
void orc_argmax(const float* logits, int rows, int V, int64_t* ids) {
  for (int r = 0; r < rows; ++r) {
    const float* l = logits + (size_t)r * V;
    int best = 0;
    for (int i = 1; i < V; ++i)
      if (l[i] > l[best]) best = i;
    ids[r] = best;
  }
}
