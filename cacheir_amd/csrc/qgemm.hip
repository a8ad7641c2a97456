// Q4_0 / Q8_0 block weights on gfx950: tiled repack, bit-exact dequant, and the
// dequant-fused MFMA GEMM  y[m][n] = sum_k x[m][k] * W[n][k].
//
// GGUF blocks (cacheir/importers/gguf.py:36,40,273-310): 32 values per block,
// Q4_0 = fp16 d + 16 bytes (byte j: element j in the low nibble, j+16 in the
// high nibble), value (nib - 8) * d; Q8_0 = fp16 d + 32 int8, value q * d.
//
// Tiled copy (made once at load, same byte count as the blocks):
//   tile (nt, Q) = rows 16*nt..16*nt+15, columns 128*Q..128*Q+127 (4 blocks).
//   quant bytes: 64 lanes x 16 B (Q4_0) or x 32 B (Q8_0); lane l = 16*g + r holds
//     row 16*nt + r, columns 128*Q + 32*j + 8*g + e (j = block in quad, e = 0..7),
//     i.e. exactly the 8-element B operand of MFMA 16x16x32 for k-step j.  Inside
//     each dword the values sit where the fp16 conversion below picks them up.
//   scales: 16 rows x 4 fp16 per tile.
// A wavefront therefore loads 1 KiB (Q4_0) contiguous per instruction.
//
// Conversion to fp16 (no table, no int->float converts):
//   Q4_0: (w & 0x000F000F) | 0x64006400 is the fp16 pair 1024+q; subtracting 1032
//   gives q-8 exactly.  (w & 0x00F000F0) | 0x64006400 is 1024+16q; times 1/16 minus
//   72 gives q-8 exactly.  w >> 8 exposes the other four nibbles the same way.
//   Q8_0: bytes xor 0x80 are q+128; (w & 0x00FF00FF) | 0x64006400 is 1024+q+128;
//   subtracting 1152 gives q exactly.
//   The MFMA B operand is these exact integers; one MFMA 16x16x32 covers exactly
//   one 32-value block, so its fp32 result is scaled by the block's d in fp32 and
//   added to the accumulator.  Products and the scale are exact in fp32, so the
//   only deviation from the fp32 reference (dequant then matmul, cpu.py:306-312)
//   is fp32 summation order.  (Rounding the weights to fp16 instead, as the
//   reference CUDA path does at cuda.py:935, misses the 2e-3 + 1e-2|y| bound at
//   k = 14336.)
//
// GEMM (qgemm_xs_kernel): workgroup = 4 wavefronts on 4*NT*16 output rows; they walk
// the quads of the workgroup's k-range in lock step and share each quad of
// activations through LDS.  grid.y splits k (fp32 partials, summed by the epilogue
// kernels); grid.z walks 16*MT-row blocks of x.
#include "common.hpp"

#include <utility>

namespace cir {
namespace {

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }

// 8 Q4_0 nibbles of one dword -> 8 fp16 values (q - 8) * 2^-12, all exact.  A nibble q
// masked in place reads as the fp16 subnormal q * 2^-24 (16q * 2^-24 for the high nibble
// of a byte); one packed FMA scales it by 2^12 (2^8) and subtracts 8 * 2^-12.  That is two
// VALU ops per pair, as many as an or-in of the exponent 1024 would need with one
// v_and_or_b32, which the compiler does not form from two literal masks.  The kernels'
// fp16 denormal mode (float_denorm_mode_16_64 = 3, the default) keeps the subnormals.
__device__ __forceinline__ f16x8 dq_q4(uint32_t w) {
  const f16x2 s12 = {(f16)4096.0f, (f16)4096.0f};
  const f16x2 s8 = {(f16)256.0f, (f16)256.0f};
  const f16x2 c8 = {(f16)-0.001953125f, (f16)-0.001953125f};  // -8 * 2^-12
  const uint32_t t = w >> 8;
  const f16x2 p0 = as_h2(w & 0x000F000Fu) * s12 + c8;
  const f16x2 p1 = as_h2(w & 0x00F000F0u) * s8 + c8;
  const f16x2 p2 = as_h2(t & 0x000F000Fu) * s12 + c8;
  const f16x2 p3 = as_h2(t & 0x00F000F0u) * s8 + c8;
  return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// 8 Q8_0 int8 values (two dwords) -> 8 exact fp16 integers q.  After the sign flip each
// byte is q + 128; one v_perm_b32 places bytes 0 and 2 (or 1 and 3) under 0x64 bytes,
// giving fp16 1024 + q + 128.  Byte selectors 4..7 pick bytes 0..3 of the first
// operand, 0..3 those of the second.
__device__ __forceinline__ f16x8 dq_q8(uint32_t w0, uint32_t w1) {
  const f16x2 c1152 = {(f16)-1152.0f, (f16)-1152.0f};
  constexpr uint32_t k64 = 0x64646464u, even = 0x00060004u, odd = 0x00070005u;
  w0 ^= 0x80808080u;
  w1 ^= 0x80808080u;
  const f16x2 p0 = as_h2(__builtin_amdgcn_perm(w0, k64, even)) + c1152;
  const f16x2 p1 = as_h2(__builtin_amdgcn_perm(w0, k64, odd)) + c1152;
  const f16x2 p2 = as_h2(__builtin_amdgcn_perm(w1, k64, even)) + c1152;
  const f16x2 p3 = as_h2(__builtin_amdgcn_perm(w1, k64, odd)) + c1152;
  return f16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// Operand position e (0..7) <- Q4_0 nibble slot nu in the dword: e = 2*(nu%4) + nu/4.
__device__ __forceinline__ int q4_elem_of_nibble(int nu) { return 2 * (nu & 3) + (nu >> 2); }
// Operand position e <- Q8_0 byte slot beta (0..7 over the two dwords): swaps 1<->2, 5<->6.
__device__ __forceinline__ int q8_elem_of_byte(int beta) {
  const int lo = beta & 3;
  const int e = (lo == 1) ? 2 : (lo == 2 ? 1 : lo);
  return (beta & 4) + e;
}

__device__ __forceinline__ int gguf_q4_nib(const uint8_t* blk, int e) {  // element e (0..31) of a block
  const uint8_t byte = blk[2 + (e & 15)];
  return (e < 16) ? (byte & 15) : (byte >> 4);
}

// Row formats (per-row scale and zero point) reuse the tile layout of the block
// format with the same code width: 4-bit codes sit like Q4_0 nibbles, 8-bit codes
// like Q8_0 bytes.  Their tiled copy holds no per-block scales; after the codes come
// fp32 scale[rows] and fp32 offset[rows] (rows padded to a multiple of 16).
__host__ __device__ constexpr bool is_row_fmt(int fmt) { return fmt == CIR_I4_ROW || fmt == CIR_I8_ROW; }
__host__ __device__ constexpr int layout_fmt(int fmt) {
  return (fmt == CIR_Q4_0 || fmt == CIR_I4_ROW) ? CIR_Q4_0 : CIR_Q8_0;
}
__host__ __device__ size_t quant_bytes_per_lane(int fmt) { return layout_fmt(fmt) == CIR_Q4_0 ? 16 : 32; }

// Accumulators of a 4-bit layout hold 2^-12 times the dot products (dq_q4's scale); each
// kernel multiplies them by kAccScale once, when its k range is done.  Scaling by a power
// of two commutes with every fp32 rounding before it (no value comes near the fp32
// subnormal range), so the results are the ones integer weights would give.
template <int FMT> inline constexpr float kAccScale = layout_fmt(FMT) == CIR_Q4_0 ? 4096.f : 1.f;
__host__ __device__ size_t block_bytes(int fmt) { return fmt == CIR_Q4_0 ? 18 : 34; }
__host__ __device__ bool valid_fmt(int fmt) {
  return fmt == CIR_Q4_0 || fmt == CIR_Q8_0 || fmt == CIR_I4_ROW || fmt == CIR_I8_ROW;
}

// ---------------------------------------------------------------- repack ----
__global__ void repack_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ qdst, uint16_t* __restrict__ ddst,
                              int fmt, int N, int K) {
  const int KQ = K / 128;
  const int NT = (N + 15) / 16;
  const long total = (long)NT * KQ * 64;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const long tile = id >> 6;
  const int Q = (int)(tile % KQ);
  const int nt = (int)(tile / KQ);
  const int r = lane & 15, g = lane >> 4;
  const int n = nt * 16 + r;
  const int nb = K / 32;
  const size_t bb = block_bytes(fmt);
  if (fmt == CIR_Q4_0) {
    uint32_t words[4];
    for (int j = 0; j < 4; ++j) {
      uint32_t w = 0;
      if (n < N) {
        const uint8_t* blk = src + ((size_t)n * nb + 4 * Q + j) * bb;
        for (int nu = 0; nu < 8; ++nu) w |= (uint32_t)gguf_q4_nib(blk, 8 * g + q4_elem_of_nibble(nu)) << (4 * nu);
      }
      words[j] = w;
    }
    uint32_t* out = reinterpret_cast<uint32_t*>(qdst + ((size_t)tile * 64 + lane) * 16);
    for (int j = 0; j < 4; ++j) out[j] = words[j];
  } else {
    uint8_t bytes[32];
    for (int j = 0; j < 4; ++j) {
      const uint8_t* blk = (n < N) ? src + ((size_t)n * nb + 4 * Q + j) * bb : nullptr;
      for (int beta = 0; beta < 8; ++beta) bytes[8 * j + beta] = blk ? blk[2 + 8 * g + q8_elem_of_byte(beta)] : 0;
    }
    uint8_t* out = qdst + ((size_t)tile * 64 + lane) * 32;
    for (int i = 0; i < 32; ++i) out[i] = bytes[i];
  }
  if (g == 0) {
    uint16_t* dd = ddst + ((size_t)tile * 16 + r) * 4;
    for (int j = 0; j < 4; ++j) {
      uint16_t dv = 0;
      if (n < N) {
        const uint8_t* blk = src + ((size_t)n * nb + 4 * Q + j) * bb;
        dv = (uint16_t)(blk[0] | (blk[1] << 8));
      }
      dd[j] = dv;
    }
  }
}

// ---------------------------------------------------------------- dequant ----
// Reference per-row asymmetric packing (quantization.py:96-139) -> tiled codes + row
// arrays.  4 bit: byte j of a row holds columns 2j (low nibble) and 2j+1 (high); the
// code stays q (the MFMA operand is q - 8).  8 bit: one byte per column; stored as
// q - 128 (the operand).  offset[row] = c0 - zero_point with c0 = 8 or 128, so
// (operand + offset) * scale = (q - zp) * scale exactly.
__global__ void repack_rows_kernel(const uint8_t* __restrict__ src, const float* __restrict__ scales,
                                   const int32_t* __restrict__ zps, uint8_t* __restrict__ qdst,
                                   float* __restrict__ rows_out, int fmt, int N, int K) {
  const int KQ = K / 128;
  const int NT = (N + 15) / 16;
  const long total = (long)NT * KQ * 64;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const long tile = id >> 6;
  const int Q = (int)(tile % KQ);
  const int nt = (int)(tile / KQ);
  const int r = lane & 15, g = lane >> 4;
  const int n = nt * 16 + r;
  if (fmt == CIR_I4_ROW) {
    const size_t row_bytes = (size_t)(K + 1) / 2;
    uint32_t* out = reinterpret_cast<uint32_t*>(qdst + ((size_t)tile * 64 + lane) * 16);
    for (int j = 0; j < 4; ++j) {
      uint32_t w = 0;
      if (n < N) {
        for (int nu = 0; nu < 8; ++nu) {
          const int col = 128 * Q + 32 * j + 8 * g + q4_elem_of_nibble(nu);
          const uint8_t byte = src[(size_t)n * row_bytes + col / 2];
          w |= (uint32_t)((col & 1) ? (byte >> 4) : (byte & 15)) << (4 * nu);
        }
      }
      out[j] = w;
    }
  } else {
    uint8_t* out = qdst + ((size_t)tile * 64 + lane) * 32;
    for (int j = 0; j < 4; ++j)
      for (int beta = 0; beta < 8; ++beta) {
        const int col = 128 * Q + 32 * j + 8 * g + q8_elem_of_byte(beta);
        out[8 * j + beta] = n < N ? (uint8_t)(src[(size_t)n * K + col] - 128u) : (uint8_t)0;
      }
  }
  if (Q == 0 && g == 0) {
    const int c0 = fmt == CIR_I4_ROW ? 8 : 128;
    rows_out[(size_t)nt * 16 + r] = n < N ? scales[n] : 0.f;
    rows_out[(size_t)NT * 16 + (size_t)nt * 16 + r] = n < N ? (float)(c0 - zps[n]) : 0.f;
  }
}

__global__ void dequant_gguf_kernel(const uint8_t* __restrict__ src, float* __restrict__ out, int fmt, int N, int K) {
  const long nblk = (long)N * (K / 32);
  const long b = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblk) return;
  const uint8_t* blk = src + b * block_bytes(fmt);
  const f16 dh = __builtin_bit_cast(f16, (uint16_t)(blk[0] | (blk[1] << 8)));
  const float d = static_cast<float>(dh);
  float* o = out + b * 32;
  if (fmt == CIR_Q4_0) {
    for (int e = 0; e < 32; ++e) o[e] = (float)(gguf_q4_nib(blk, e) - 8) * d;
  } else {
    for (int e = 0; e < 32; ++e) o[e] = (float)(int8_t)blk[2 + e] * d;
  }
}

__global__ void dequant_tiled_kernel(const uint8_t* __restrict__ q, const void* __restrict__ scales_any,
                                     float* __restrict__ out, int fmt, int N, int K) {
  // One thread per (tile, lane): 32 values (4 k-steps x 8).
  const int KQ = K / 128;
  const int NT = (N + 15) / 16;
  const long total = (long)NT * KQ * 64;
  const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= total) return;
  const int lane = (int)(id & 63);
  const long tile = id >> 6;
  const int Q = (int)(tile % KQ), nt = (int)(tile / KQ);
  const int r = lane & 15, g = lane >> 4;
  const int n = nt * 16 + r;
  if (n >= N) return;
  const uint16_t* dsc = static_cast<const uint16_t*>(scales_any);
  const float* rsc = static_cast<const float*>(scales_any);
  for (int j = 0; j < 4; ++j) {
    // block formats: value = operand * d; row formats: (operand + offset) * scale
    float d, off = 0.f;
    if (is_row_fmt(fmt)) {
      d = rsc[n];
      off = rsc[(size_t)NT * 16 + n];
    } else {
      d = static_cast<float>(__builtin_bit_cast(f16, dsc[((size_t)tile * 16 + r) * 4 + j]));
    }
    float* o = out + (size_t)n * K + 128 * Q + 32 * j + 8 * g;
    if (layout_fmt(fmt) == CIR_Q4_0) {
      const uint32_t w = reinterpret_cast<const uint32_t*>(q + ((size_t)tile * 64 + lane) * 16)[j];
      for (int nu = 0; nu < 8; ++nu)
        o[q4_elem_of_nibble(nu)] = ((float)((int)((w >> (4 * nu)) & 15) - 8) + off) * d;
    } else {
      const uint8_t* bytes = q + ((size_t)tile * 64 + lane) * 32 + 8 * j;
      for (int beta = 0; beta < 8; ++beta) o[q8_elem_of_byte(beta)] = ((float)(int8_t)bytes[beta] + off) * d;
    }
  }
}

// ------------------------------------------------------------------ GEMM -----
// One quad (128 columns) of operands for one wavefront: NT weight tiles (codes and
// scales) and the MT activation tiles as MFMA A operands.
template <int FMT, int NT, int MT>
struct Stage {
  static constexpr int LB = (layout_fmt(FMT) == CIR_Q4_0) ? 1 : 2;  // 16-byte loads per lane per weight tile
  uint4 w[NT][LB];
  uint2 d[NT];
  f16x8 x[MT][4];
};

// Exact weights ((q - 8) * 2^-12 for Q4_0, q for Q8_0) feed one MFMA per 32-value
// block; the block's fp32 result is scaled by d in fp32 and accumulated, in block order.
// The MFMAs of block j + 1 are issued before the scale FMAs of block j (two sets of
// block results in registers), so each FMA waits on an MFMA issued a block earlier:
// config-4 step 3.452-3.463 -> 3.442-3.457 ms (three alternated pairs), batch 1 unchanged.
// MR: accumulator rows per lane group that are scaled (lane group g holds rows 4g .. 4g+3 of a
// tile; at m = 1 only row 0 is real, and MR = 1 saves three of every four scale FMAs).
template <int FMT, int NT, int MT, int MR = 4>
__device__ __forceinline__ void compute_stage(const Stage<FMT, NT, MT>& st, f32x4 (&acc)[MT][NT]) {
  auto wfrag = [&](int b, int j) __attribute__((always_inline)) {
    f16x8 wb;
    if constexpr (layout_fmt(FMT) == CIR_Q4_0) {
      const uint4 v = st.w[b][0];
      wb = dq_q4((j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w);
    } else {
      const uint4 v = st.w[b][j >> 1];
      wb = dq_q8((j & 1) ? v.z : v.x, (j & 1) ? v.w : v.y);
    }
    return wb;
  };
  if constexpr (is_row_fmt(FMT)) {
    // one scale per row: integers accumulate over all k in the MFMA itself
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int b = 0; b < NT; ++b) {
        const f16x8 wb = wfrag(b, j);
#pragma unroll
        for (int a = 0; a < MT; ++a) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(st.x[a][j], wb, acc[a][b], 0, 0, 0);
      }
  } else {
    f32x4 c[2][MT][NT];
    auto mfmas = [&](int j, f32x4 (&cc)[MT][NT]) __attribute__((always_inline)) {
#pragma unroll
      for (int b = 0; b < NT; ++b) {
        const f16x8 wb = wfrag(b, j);
#pragma unroll
        for (int a = 0; a < MT; ++a)
          cc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(st.x[a][j], wb, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      }
    };
    auto fmas = [&](int j, const f32x4 (&cc)[MT][NT]) __attribute__((always_inline)) {
#pragma unroll
      for (int b = 0; b < NT; ++b) {
        const uint32_t dw = (j < 2) ? st.d[b].x : st.d[b].y;
        const float dj = static_cast<float>(__builtin_bit_cast(f16, (uint16_t)((j & 1) ? (dw >> 16) : (dw & 0xFFFFu))));
#pragma unroll
        for (int a = 0; a < MT; ++a)
#pragma unroll
          for (int r = 0; r < MR; ++r) acc[a][b][r] = fmaf(dj, cc[a][b][r], acc[a][b][r]);
      }
    };
    mfmas(0, c[0]);
    mfmas(1, c[1]);
    fmas(0, c[0]);
    mfmas(2, c[0]);
    fmas(1, c[1]);
    mfmas(3, c[1]);
    fmas(2, c[0]);
    fmas(3, c[1]);
  }
}

// Row sums of the activation quad (row formats): sx[a] += x[16a + 4*lg + r][quad] . 1,
// by MFMA against an all-ones B operand, so the C layout matches the accumulators'.
template <int MT>
__device__ __forceinline__ void row_sums(const f16x8 (&x)[MT][4], f32x4 (&sx)[MT]) {
  const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int a = 0; a < MT; ++a) sx[a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[a][j], ones, sx[a], 0, 0, 0);
}

// Dense fp32: one wavefront per output row n, lanes over k; all m rows.
__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ x, int ldx, const float* __restrict__ w,
                                                       float* __restrict__ part, int M, int N, int K, int kc) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + wave;
  if (n >= N) return;
  const int split = blockIdx.y;
  const int k0 = split * kc, k1 = min(K, k0 + kc);
  const float* wr = w + (size_t)n * K;
  for (int m = 0; m < M; ++m) {
    const float* xr = x + (size_t)m * ldx;
    float s = 0.f;
    for (int k = k0 + lane; k < k1; k += 64) s = fmaf(xr[k], wr[k], s);
    s = wave_sum(s);
    if (lane == 0) part[((size_t)split * M + m) * N + n] = s;
  }
}

// ---------------------------------------------------------- x-shared GEMM ---
// The four wavefronts of a workgroup own different output tiles (NT each) and walk
// the same k-quads in lock step, so each quad of activations is read from L2 once
// per workgroup (cooperatively, 16 B per thread per 16-row tile) and shared through
// LDS, instead of once per wavefront.  Weights stream through a ring of DW stages
// per wavefront; each stage's activation loads are issued before its weight loads,
// so waiting for the activations of quad i+1 never waits for weights issued later.
// One workgroup barrier per quad: it publishes the activation slot written for
// quad i+1 and releases the slot read for quad i.
constexpr int kXsRowBytes = 272;  // 128 fp16 + 16 B pad: the 16 rows of a fragment read hit different banks

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // plain vector: no struct memcpy, stays in VGPRs

template <int MT>
struct XsChunk {  // this thread's share of one quad of activations
  u32x4 v[MT];
};

// KG k-groups: a workgroup holds KG groups of four wavefronts on the same output
// tiles; group g takes quads q0 + g, q0 + g + KG, ... of the split, so each SIMD runs
// KG wavefronts and one wavefront's dequant/MFMA work overlaps another's loads.  The
// groups' accumulators are summed through LDS in group order at the end.
// EPI 0: store fp32 split-k partials part[split][m][n].
// EPI 1 (SwiGLU, one split): the weight tiles alternate gate / up (tile 2c = gate
// rows 16c.., tile 2c+1 = the matching up rows), so a wavefront with NT = 2 holds
// both accumulators of 16 intermediate columns and writes silu(g) * u to
// out[m][N/2] (type TO) -- the SwiGLU of cpu.py:266-279 without a partials pass.
// EPI 2 (greedy head, one split): no logits are stored; each wavefront writes, per
// row, the best (value, column) of its NT*16 columns to cand_v / cand_i
// [m][wavefront] (part and act reinterpreted), reduced by argmax_cand_kernel.
template <int FMT, int NT, int MT, int DW, int EPI = 0, typename TO = float, int KG = 1, int MR = 4>
__global__ __launch_bounds__(256 * KG) void qgemm_xs_kernel(const f16* __restrict__ x, int ldx,
                                                       const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                       float* __restrict__ part, int M, int N, int K,
                                                       int quads_per_split, TO* __restrict__ act = nullptr) {
  static_assert(EPI != 1 || NT == 2, "the SwiGLU epilogue pairs tile 2c (gate) with 2c+1 (up)");
  constexpr int LB = Stage<FMT, NT, MT>::LB;
  constexpr int kSlot = 16 * MT * kXsRowBytes;  // one quad of activations
  // after the k loop the same memory holds groups 1..KG-1's accumulators (and row sums)
  constexpr int kRed = (KG - 1) * 4 * (MT * NT + (is_row_fmt(FMT) ? MT : 0)) * 4 * 64 * (int)sizeof(float);
  __shared__ __align__(16) uint8_t smem[(2 * KG * kSlot > kRed) ? 2 * KG * kSlot : kRed];
  const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kg = wave_all >> 2, wave = wave_all & 3;
  const int tid = threadIdx.x & 255;  // thread index inside the k-group
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int KQ = K / 128;
  const int NTILES = (N + 15) / 16;
  const int nt0 = (blockIdx.x * 4 + wave) * NT;  // this wavefront's first tile
  const int split = blockIdx.y;
  const int m0 = blockIdx.z * 16 * MT;
  const int q0 = split * quads_per_split + kg;
  const int nq = quads_per_split / KG;  // this group's quads (the host makes KG divide quads_per_split)

  // Cooperative activation chunk of this thread: row r = c / 16, 16-byte column c % 16.
  const f16* xsrc[MT];
  int xdst[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    const int c = tid + 256 * u;
    const int r = c >> 4, col = c & 15;
    xsrc[u] = x + (size_t)min(m0 + r, M - 1) * ldx + 8 * col;  // rows past M re-read row M-1 (never stored)
    xdst[u] = r * kXsRowBytes + 16 * col;
  }
  const uint4* wbase[NT];
  const uint2* dbase[NT];
#pragma unroll
  for (int b = 0; b < NT; ++b) {
    const size_t tile0 = (size_t)min(nt0 + b, NTILES - 1) * KQ;
    wbase[b] = reinterpret_cast<const uint4*>(wq) + (tile0 * 64 + lane) * LB;
    dbase[b] = reinterpret_cast<const uint2*>(wd) + tile0 * 16 + li;
  }

  struct WS {
    uint4 w[NT][LB];
    uint2 d[NT];
  };
  WS ws[DW];
  XsChunk<MT> xc[DW];
  // (always_inline: a ring slot index must fold to a constant, or the rings go to scratch)
  auto issue = [&](int slot_w, int idx) __attribute__((always_inline)) {  // stage idx (clamped to the last quad)
    const int Q = q0 + KG * min(idx, nq - 1);
#pragma unroll
    for (int u = 0; u < MT; ++u) xc[slot_w].v[u] = *reinterpret_cast<const u32x4*>(xsrc[u] + 128 * Q);
#pragma unroll
    for (int b = 0; b < NT; ++b) {
      const uint4* src = wbase[b] + (size_t)Q * (64 * LB);
#pragma unroll
      for (int c = 0; c < LB; ++c) ws[slot_w].w[b][c] = src[c];
      if constexpr (!is_row_fmt(FMT)) ws[slot_w].d[b] = dbase[b][(size_t)Q * 16];
    }
  };
  auto put_x = [&](int slot_x, const XsChunk<MT>& ch) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < MT; ++u) *reinterpret_cast<u32x4*>(&smem[(slot_x * KG + kg) * kSlot + xdst[u]]) = ch.v[u];
  };
  auto barrier = [] { __syncthreads(); };

  f32x4 acc[MT][NT];
  f32x4 sx[MT];  // row formats: sums of this split's activations, per output row
#pragma unroll
  for (int a = 0; a < MT; ++a) {
    sx[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](const WS& st, int slot_x) __attribute__((always_inline)) {
    Stage<FMT, NT, MT> sg;  // reuse compute_stage: fragments from LDS, weights from the ring
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sg.x[a][j] = *reinterpret_cast<const f16x8*>(
            &smem[(slot_x * KG + kg) * kSlot + (16 * a + li) * kXsRowBytes + 64 * j + 16 * lg]);
#pragma unroll
    for (int b = 0; b < NT; ++b) {
#pragma unroll
      for (int c = 0; c < LB; ++c) sg.w[b][c] = st.w[b][c];
      if constexpr (!is_row_fmt(FMT)) sg.d[b] = st.d[b];
    }
    compute_stage<FMT, NT, MT, MR>(sg, acc);
    if constexpr (is_row_fmt(FMT)) row_sums(sg.x, sx);
  };

  // Ring slots are template arguments (std::integer_sequence), so every ring access
  // has a compile-time index and the rings stay in registers.
  auto each = [&](auto&& f) __attribute__((always_inline)) {
    [&]<int... S>(std::integer_sequence<int, S...>) { (f.template operator()<S>(), ...); }(
        std::make_integer_sequence<int, DW>{});
  };
  // Prologue: stages 0 .. DW-1 in flight, activations of quad 0 in LDS slot 0.
  each([&]<int S>() { issue(S, S); });
  put_x(0, xc[0]);
  barrier();
  // Steady state: at index i + S publish x(i+S+1), compute quad i+S, then refill
  // ring slot S with stage i+S+DW.  The LDS slot of quad idx is idx & 1.
  int i = 0;
  for (; i + DW <= nq; i += DW) {
    each([&]<int S>() {
      put_x((i + S + 1) & 1, xc[(S + 1) % DW]);
      compute(ws[S], (i + S) & 1);
      issue(S, i + S + DW);
      barrier();
    });
  }
  each([&]<int S>() {
    if (S < DW - 1 && i + S < nq) {
      put_x((i + S + 1) & 1, xc[(S + 1) % DW]);
      compute(ws[S], (i + S) & 1);
      barrier();
    }
  });
  if constexpr (kAccScale<FMT> != 1.f) {
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[a][b] *= kAccScale<FMT>;
  }

  if constexpr (KG > 1) {
    // The loop ended on a barrier after the last LDS read.  Groups 1.. park their
    // accumulators (and row sums) in LDS; group 0 adds them in group order.
    float* red = reinterpret_cast<float*>(smem);
    constexpr int kVals = MT * NT + (is_row_fmt(FMT) ? MT : 0);  // f32x4 per lane
    auto slot = [&](int g, int v, int r) { return ((((g - 1) * 4 + wave) * kVals + v) * 4 + r) * 64 + lane; };
    if (kg > 0) {
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int b = 0; b < NT; ++b) red[slot(kg, a * NT + b, r)] = acc[a][b][r];
          if constexpr (is_row_fmt(FMT)) red[slot(kg, MT * NT + a, r)] = sx[a][r];
        }
    }
    barrier();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KG; ++g)
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
          for (int b = 0; b < NT; ++b) acc[a][b][r] += red[slot(g, a * NT + b, r)];
          if constexpr (is_row_fmt(FMT)) sx[a][r] += red[slot(g, MT * NT + a, r)];
        }
  }
  if constexpr (is_row_fmt(FMT)) {
    // w = (c - zp) * s with c the stored code: acc holds sum x*c over this split, so
    // the split's share of y is s * (acc + (c0 - zp) * sum x), c0 - zp = offset[row].
    const float* rscale = reinterpret_cast<const float*>(wd);
    const float* roff = rscale + (size_t)NTILES * 16;
#pragma unroll
    for (int b = 0; b < NT; ++b) {
      const int n = min(nt0 + b, NTILES - 1) * 16 + li;
      const float sc = rscale[n], of = roff[n];
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[a][b][r] = sc * fmaf(of, sx[a][r], acc[a][b][r]);
    }
  }
  if constexpr (EPI == 2) {
    float* cand_v = part;
    int* cand_i = reinterpret_cast<int*>(act);
    const int wv_global = blockIdx.x * 4 + wave;
    const int W = gridDim.x * 4;
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int b = 0; b < NT; ++b) {
          const int n = (nt0 + b) * 16 + li;
          if (nt0 + b < NTILES && n < N) argmax_better(bv, bi, acc[a][b][r], n);
        }
        // the 16 lanes of this row group (same lg) hold 16 different columns
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          argmax_better(bv, bi, ov, oi);
        }
        const int m = m0 + 16 * a + 4 * lg + r;
        if (li == 0 && m < M) {
          cand_v[(size_t)m * W + wv_global] = bv;
          cand_i[(size_t)m * W + wv_global] = bi;
        }
      }
  } else if constexpr (EPI == 1) {
    const int inter = N / 2;
    const int col = (nt0 >> 1) * 16 + li;
    if (nt0 + 1 < NTILES && col < inter) {
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * a + 4 * lg + r;
          const float g = acc[a][0][r], u = acc[a][1][r];
          if (m < M) act[(size_t)m * inter + col] = static_cast<TO>(as_f32_value((g / (1.0f + expf(-g))) * u));
        }
    }
  } else {
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) {
        const int n = (nt0 + b) * 16 + li;
        if (nt0 + b < NTILES && n < N) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * a + 4 * lg + r;
            if (m < M) part[((size_t)split * M + m) * N + n] = acc[a][b][r];
          }
        }
      }
  }
}

// ------------------------------------------------------------------ GEMV -----
typedef __amdgpu_buffer_rsrc_t rsrc_t;
// Raw buffer resource over [p, p + bytes) (gfx9 descriptor word 3: raw byte-addressed
// loads, out-of-range lanes read 0).
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ uint4 buf16(rsrc_t r, uint32_t voff, uint32_t soff) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
  return uint4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ uint2 buf8(rsrc_t r, uint32_t voff, uint32_t soff) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
  return uint2{v.x, v.y};
}
// 16 bytes per lane from the buffer straight into LDS: lane l's bytes land at lds + 16 l.
// (A device function, not a lambda: kernel lambdas are also compiled for the host,
// where the builtin does not exist, and the host pass then drops the kernel's stub.)
__device__ __forceinline__ void buf16_to_lds(rsrc_t r, uint8_t* lds, uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// ------------------------------------------------------------- large m ------
// m > 32 (qgemm_xl_kernel): a workgroup of 4 wavefronts covers 8 weight tiles (128
// output columns, 2 per wavefront) and 16*MT activation rows, so each weight tile is
// read once per 16*MT rows (the m <= 32 kernel reads it once per 32).  A quad of
// activations (16*MT rows x 128 columns fp16, 4 KiB per 16 rows) goes straight to
// LDS by buffer DMA (no registers), double-buffered, one barrier per quad.  Chunk g
// (16 B) of row r sits in slot g ^ (r & 15) of the row's 256 B, so the 16 rows of a
// fragment read hit 16 different bank groups.  Weights stream through a ring of
// DW + 1 slots as in the GEMV.  Per tile and quad the blocks are scaled and summed in
// the m <= 32 kernel's order, so for the same split both give the same bits.
// EPI 0: fp32 split-k partials part[split][m][n]; EPI 1: SwiGLU over interleaved
// gate/up tiles (one split), out[m][N/2] in type TO; EPI 2: greedy-head candidates
// (one split), the best column of each wavefront's 32 and row: value in part, index in
// act (as int), at [m][blockIdx.x * W + wave], for argmax_cand_kernel.
// IL: ask the scheduler to interleave one MFMA with five VALU instructions (the block scale FMAs and dequant)
// instead of its own two-MFMA / eight-FMA order; PF: convert each block scale to fp32 once and scale with plain
// fp32 FMAs (the compiler otherwise reads the fp16 scale in every v_fma_mix_f32; same values, same bits).  See
// launch_qgemm_xl for where each pays.
template <int FMT, int MT, int DW, int EPI = 0, typename TO = float, int W = 4, bool IL = false, bool PF = false>
__global__ __launch_bounds__(64 * W) void qgemm_xl_kernel(const f16* __restrict__ x, int ldx,
                                                     const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                     float* __restrict__ part, int M, int N, int K, int nq,
                                                     TO* __restrict__ act = nullptr) {
  static_assert(EPI >= 0 && EPI <= 2, "large-m GEMM epilogues: partials, SwiGLU or argmax candidates");
  constexpr int NT = 2;
  // Issue order of the block MFMAs and scale FMAs: pipelined by one block for the greedy head (Qwen2-7B lm_head
  // at m = 128: 255.3-255.9 -> 245.6-246.2 us, alternated on one box); elsewhere it measured no better (2048-row
  // gate|up + SwiGLU within noise) or worse (with the interleave hint: config 5's QKV 14.2 -> 15.1 us).
  constexpr bool kPipe = !is_row_fmt(FMT) && EPI == 2;
  constexpr int LB = Stage<FMT, NT, 1>::LB;
  constexpr int kSlot = 16 * MT * 256;  // bytes of one quad of activations
  __shared__ __align__(16) uint8_t smem0[kSlot];  // two arrays, not one: the compiler then
  __shared__ __align__(16) uint8_t smem1[kSlot];  // lets reads of one run while DMA fills the other
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int KQ = K / 128, NTILES = (N + 15) / 16;
  const int nt0 = (blockIdx.x * W + wave) * NT;
  const int split = blockIdx.y;
  const int m0 = blockIdx.z * 16 * MT;
  const int q0 = split * nq;
  const int nqs = min(nq, KQ - q0);  // quads of this split (the last may hold fewer)

  // Activation DMA: instruction u (0..XU-1) of wavefront w fills LDS bytes
  // [(w*XU + u) KiB, +1 KiB) of a slot, 16 B per lane: row r = 4 (w*XU + u) + lane/16,
  // slot s = lane % 16 holds chunk s ^ (r & 15).  Rows past M re-read row M-1.
  constexpr int XU = 4 * MT / W;  // KiB of a quad each wavefront brings in
  static_assert(XU * W == 4 * MT, "the wavefronts split a quad of activations evenly");
  const rsrc_t rx = make_rsrc(x, (uint32_t)((size_t)M * ldx * 2));
  uint32_t xoff[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int r = 4 * (wave * XU + u) + (lane >> 4);
    const int g = (lane & 15) ^ (r & 15);
    xoff[u] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)ldx * 2u + 16u * g;
  }
  auto dma_x = [&](int slot, int Q) __attribute__((always_inline)) {
    uint8_t* sm = slot ? smem1 : smem0;
#pragma unroll
    for (int u = 0; u < XU; ++u)
      buf16_to_lds(rx, sm + (wave * XU + u) * 1024, xoff[u], 256u * (uint32_t)(q0 + Q));
  };

  const uint32_t ntiles_total = (uint32_t)NTILES * KQ;
  const rsrc_t rw = make_rsrc(wq, ntiles_total * 1024u * LB);
  const rsrc_t rd = make_rsrc(wd, is_row_fmt(FMT) ? 0u : ntiles_total * 128u);
  uint32_t tb[NT];
#pragma unroll
  for (int b = 0; b < NT; ++b) tb[b] = (uint32_t)min(nt0 + b, NTILES - 1) * KQ + q0;
  const uint32_t vw = (uint32_t)lane * 16u * LB, vd = (uint32_t)li * 8u;
  struct WS {
    uint4 w[NT][LB];
    uint2 d[NT];
  };
  constexpr int R = DW + 1;
  WS ws[R];
  auto issue = [&](int slot, int idx) __attribute__((always_inline)) {  // quad idx, clamped to the last
    const uint32_t Q = (uint32_t)min(idx, nqs - 1);
#pragma unroll
    for (int b = 0; b < NT; ++b) {
#pragma unroll
      for (int c = 0; c < LB; ++c) ws[slot].w[b][c] = buf16(rw, vw + 16u * c, (tb[b] + Q) * 1024u * LB);
      if constexpr (!is_row_fmt(FMT)) ws[slot].d[b] = buf8(rd, vd, (tb[b] + Q) * 128u);
    }
  };
  auto each = [&]<int C>(auto&& f) __attribute__((always_inline)) {
    [&]<int... S>(std::integer_sequence<int, S...>) { (f.template operator()<S>(), ...); }(
        std::make_integer_sequence<int, C>{});
  };

  f32x4 acc[MT][NT];
  f32x4 sx[MT];  // row formats: activation sums of this split
#pragma unroll
  for (int a = 0; a < MT; ++a) {
    sx[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NT; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  int xo[4];  // swizzled byte offset of chunk 4j + lg in row 16a + li (li & 15 = li)
#pragma unroll
  for (int j = 0; j < 4; ++j) xo[j] = li * 256 + (((4 * j + lg) ^ li) << 4);

  auto compute = [&](const WS& st, int xslot) __attribute__((always_inline)) {
    f16x8 wb[NT][4];
    float dj[NT][4];
#pragma unroll
    for (int b = 0; b < NT; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (layout_fmt(FMT) == CIR_Q4_0) {
          const uint4 v = st.w[b][0];
          wb[b][j] = dq_q4((j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w);
        } else {
          const uint4 v = st.w[b][j >> 1];
          wb[b][j] = dq_q8((j & 1) ? v.z : v.x, (j & 1) ? v.w : v.y);
        }
        if constexpr (!is_row_fmt(FMT)) {
          const uint32_t dw = (j < 2) ? st.d[b].x : st.d[b].y;
          dj[b][j] = static_cast<float>(__builtin_bit_cast(f16, (uint16_t)((j & 1) ? (dw >> 16) : (dw & 0xFFFFu))));
          if constexpr (PF) asm volatile("" : "+v"(dj[b][j]));  // keeps the conversion out of the FMAs
        }
      }
    const uint8_t* xq = xslot ? smem1 : smem0;
#pragma unroll
    for (int a = 0; a < MT; ++a) {
      f16x8 xf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xf[j] = *reinterpret_cast<const f16x8*>(xq + a * 4096 + xo[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (is_row_fmt(FMT)) {
#pragma unroll
          for (int b = 0; b < NT; ++b) acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wb[b][j], acc[a][b], 0, 0, 0);
          const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
          sx[a] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], ones, sx[a], 0, 0, 0);
        } else if constexpr (!kPipe) {
          f32x4 c[NT];
#pragma unroll
          for (int b = 0; b < NT; ++b)
            c[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wb[b][j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
          for (int b = 0; b < NT; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[a][b][r] = fmaf(dj[b][j], c[b][r], acc[a][b][r]);
        }
      }
      if constexpr (kPipe) {  // block j+1's MFMAs before block j's scale FMAs; same arithmetic and order
        f32x4 c[2][NT];
        auto mf = [&](int j, f32x4 (&cc)[NT]) __attribute__((always_inline)) {
#pragma unroll
          for (int b = 0; b < NT; ++b)
            cc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wb[b][j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        };
        auto fm = [&](int j, const f32x4 (&cc)[NT]) __attribute__((always_inline)) {
#pragma unroll
          for (int b = 0; b < NT; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[a][b][r] = fmaf(dj[b][j], cc[b][r], acc[a][b][r]);
        };
        mf(0, c[0]);
        mf(1, c[1]);
        fm(0, c[0]);
        mf(2, c[0]);
        fm(1, c[1]);
        mf(3, c[1]);
        fm(2, c[0]);
        fm(3, c[1]);
      }
    }
    if constexpr (IL) {
#pragma unroll
      for (int i = 0; i < MT * 4 * NT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
      }
    }
  };

  auto barrier = [] { __syncthreads(); };
  // Prologue: activations of quad 0 (slot 0) and weight stages 0 .. DW-1 in flight.
  dma_x(0, 0);
  each.template operator()<DW>([&]<int S>() { issue(S, S); });
  barrier();  // (the compiler waits for this wavefront's DMA before the barrier)
  // Stage i: DMA quad i+1 into the other slot, compute quad i, refill the ring, then the
  // barrier that publishes quad i+1 (and frees slot i & 1).  The wait before the barrier
  // covers the DMA and the loads issued before it, not the weights issued after it.
  // An even ring length keeps i even, so each step's slot S & 1 is known at compile time
  // and the DMA can go out first: the compute reads the other array, which the compiler
  // does not wait on.  (With one array, or a slot known only at run time, it waits for
  // the DMA and every load before it; an odd ring would need 2R steps unrolled, which
  // spilled.)
  static_assert(R % 2 == 0, "the slot of each step is fixed only for an even ring");
  int i = 0;
#pragma nounroll
  for (; i + R <= nqs; i += R) {
    each.template operator()<R>([&]<int S>() {
      dma_x((S + 1) & 1, min(i + S + 1, nqs - 1));
      compute(ws[S], S & 1);
      issue((S + DW) % R, i + S + DW);
      barrier();
    });
  }
  each.template operator()<DW>([&]<int S>() {  // at most DW quads are left, in ring slots 0 .. DW-1 (i even)
    if (i + S < nqs) {
      if (i + S + 1 < nqs) dma_x((S + 1) & 1, i + S + 1);
      compute(ws[S], S & 1);
      barrier();
    }
  });
  if constexpr (kAccScale<FMT> != 1.f) {
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) acc[a][b] *= kAccScale<FMT>;
  }

  if constexpr (is_row_fmt(FMT)) {
    const float* rscale = reinterpret_cast<const float*>(wd);
    const float* roff = rscale + (size_t)NTILES * 16;
#pragma unroll
    for (int b = 0; b < NT; ++b) {
      const int n = min(nt0 + b, NTILES - 1) * 16 + li;
      const float sc = rscale[n], of = roff[n];
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[a][b][r] = sc * fmaf(of, sx[a][r], acc[a][b][r]);
    }
  }
  if constexpr (EPI == 2) {
    float* cand_v = part;
    int* cand_i = reinterpret_cast<int*>(act);
    const int wv_global = blockIdx.x * W + wave;
    const int WT = gridDim.x * W;
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int b = 0; b < NT; ++b) {
          const int n = (nt0 + b) * 16 + li;
          if (nt0 + b < NTILES && n < N) argmax_better(bv, bi, acc[a][b][r], n);
        }
        // the 16 lanes of this row group (same lg) hold 16 different columns
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
          const float ov = __shfl_xor(bv, off, 64);
          const int oi = __shfl_xor(bi, off, 64);
          argmax_better(bv, bi, ov, oi);
        }
        const int m = m0 + 16 * a + 4 * lg + r;
        if (li == 0 && m < M) {
          cand_v[(size_t)m * WT + wv_global] = bv;
          cand_i[(size_t)m * WT + wv_global] = bi;
        }
      }
  } else if constexpr (EPI == 1) {
    const int inter = N / 2;
    const int col = (nt0 >> 1) * 16 + li;
    if (nt0 + 1 < NTILES && col < inter) {
#pragma unroll
      for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * a + 4 * lg + r;
          const float g = acc[a][0][r], u = acc[a][1][r];
          if (m < M) act[(size_t)m * inter + col] = static_cast<TO>(as_f32_value((g / (1.0f + expf(-g))) * u));
        }
    }
  } else {
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
      for (int b = 0; b < NT; ++b) {
        const int n = (nt0 + b) * 16 + li;
        if (nt0 + b < NTILES && n < N) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = m0 + 16 * a + 4 * lg + r;
            if (m < M) part[((size_t)split * M + m) * N + n] = acc[a][b][r];
          }
        }
      }
  }
}

// Balanced large m (qgemm_xw_kernel): one workgroup of 4 wavefronts per CU, each
// workgroup owning a contiguous run of 1..5 tile pairs (gate/up pairs for SwiGLU) and all
// 16*MT rows of its row block, so the launch is one round over the CUs with every CU's
// share of the columns within one pair of the mean (the large-m kernel's fixed 128-column
// groups leave 2 or 3 workgroups per CU).  Per quad the weight codes and scales of the
// run and the activations all go to LDS by buffer DMA, double-buffered in two separate
// arrays so the compiler lets the LDS reads of one slot overlap the DMA into the other.
// Wavefront w computes pair w over all rows and, in a 5-pair run, row tiles w*MT/4 ..
// (w+1)*MT/4 - 1 of the fifth pair: each dequantized fragment feeds MT (or MT/4) MFMAs,
// and in 4- and 5-pair runs the four wavefronts have the same MFMA count.  Per tile, quad and block the arithmetic is the
// large-m kernel's in the same order, so both give the same bits over one split.  The
// epilogue is the SwiGLU over interleaved gate/up tiles, out[m][N/2] in type TO (one
// split, the whole of k).  Block formats only.
constexpr int kXwPairs = 5;
template <int FMT>
inline constexpr int kXwTileBytes = 1024 * Stage<FMT, 1, 1>::LB;  // codes of one tile and quad
// One slot: activations (16*MT rows x 256 B), codes of up to 10 tiles, then 2 KiB of
// scales (two whole DMA instructions: tiles 0-7 and 8-9, the rest of the second unused).
template <int FMT, int MT>
inline constexpr int kXwSlot = 16 * MT * 256 + 2 * kXwPairs * kXwTileBytes<FMT> + 2048;

template <int FMT, int MT, int W>
__device__ __forceinline__ void xw_dma(uint8_t* slot, rsrc_t rx, rsrc_t rw, rsrc_t rd,
                                       const uint32_t (&xoff)[4 * MT / W], int wave, int lane, int t0, int ntl, int KQ,
                                       int Q) {
  constexpr int TB = kXwTileBytes<FMT>, LB = TB / 1024;
  constexpr int XB = 16 * MT * 256, XU = 4 * MT / W;
  // activations: wavefront w brings KiB w*XU .. w*XU+XU-1 of the quad (rows 4 KiB-index + lane/16)
#pragma unroll
  for (int u = 0; u < XU; ++u) buf16_to_lds(rx, slot + (wave * XU + u) * 1024, xoff[u], 256u * (uint32_t)Q);
  // codes: instruction i = tile i / LB, KiB i % LB; wavefront w takes i = w, w + W, ...
#pragma unroll
  for (int v = 0; v < (2 * kXwPairs * LB + W - 1) / W; ++v) {
    const int i = wave + W * v;
    if (i < ntl * LB) {
      const int t = i / LB, c = i - t * LB;
      buf16_to_lds(rw, slot + XB + t * TB + c * 1024, (uint32_t)lane * 16u + 1024u * c,
                   ((uint32_t)(t0 + t) * KQ + Q) * (uint32_t)TB);
    }
  }
  // scales: 128 B per tile; lane l of wavefront w (w < 2) brings 16 B of tile 8w + l/8
  // (lanes past the run repeat its last tile into bytes nothing reads)
  if (wave < 2 && 8 * wave < ntl) {
    const int t = min(8 * wave + (lane >> 3), ntl - 1);
    buf16_to_lds(rd, slot + XB + 2 * kXwPairs * TB + wave * 1024,
                 ((uint32_t)(t0 + t) * KQ + Q) * 128u + 16u * (lane & 7), 0u);
  }
}

constexpr int kXwWaves = 4;
template <int FMT, int MT, typename TO>
__global__ __launch_bounds__(64 * kXwWaves) void qgemm_xw_kernel(const f16* __restrict__ x, int ldx,
                                                     const uint8_t* __restrict__ wq, const uint16_t* __restrict__ wd,
                                                     int M, int N, int K, TO* __restrict__ act) {
  static_assert(!is_row_fmt(FMT), "block formats only");
  constexpr int W = kXwWaves;
  static_assert(MT % W == 0, "the fifth pair's rows split over the wavefronts");
  constexpr int TB = kXwTileBytes<FMT>, LB = TB / 1024;
  constexpr int XB = 16 * MT * 256, WB = 2 * kXwPairs * TB, SLOT = kXwSlot<FMT, MT>;
  constexpr int XU = 4 * MT / W;   // KiB of a quad's activations each wavefront brings in
  constexpr int MT5 = MT / W;      // row tiles of the fifth pair per wavefront
  __shared__ __align__(16) uint8_t slot_a[SLOT];
  __shared__ __align__(16) uint8_t slot_b[SLOT];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int KQ = K / 128, NTILES = (N + 15) / 16, NP = (NTILES + 1) / 2;
  const int p0 = (int)((long)blockIdx.x * NP / gridDim.x);
  const int cnt = (int)((long)(blockIdx.x + 1) * NP / gridDim.x) - p0;  // 1..5 pairs (host-checked)
  const int t0 = 2 * p0, ntl = min(2 * cnt, NTILES - t0);
  const int q0 = 0, nqs = KQ;
  const int m0 = blockIdx.z * 16 * MT;

  const rsrc_t rx = make_rsrc(x, (uint32_t)((size_t)M * ldx * 2));
  const uint32_t ntiles_total = (uint32_t)NTILES * KQ;
  const rsrc_t rw = make_rsrc(wq, ntiles_total * (uint32_t)TB);
  const rsrc_t rd = make_rsrc(wd, ntiles_total * 128u);
  uint32_t xoff[XU];
#pragma unroll
  for (int u = 0; u < XU; ++u) {
    const int r = 4 * (wave * XU + u) + (lane >> 4);
    const int g = (lane & 15) ^ (r & 15);
    xoff[u] = (uint32_t)min(m0 + r, M - 1) * (uint32_t)ldx * 2u + 16u * g;
  }

  const bool own = wave < cnt;          // pair `wave` of the run, all rows
  const bool fifth = cnt == kXwPairs;    // pair 4, row tiles wave*MT5 .. of it
  f32x4 acc[MT][2], acc5[MT5][2];
#pragma unroll
  for (int a = 0; a < MT; ++a) acc[a][0] = acc[a][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int a = 0; a < MT5; ++a) acc5[a][0] = acc5[a][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  int xo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) xo[j] = li * 256 + (((4 * j + lg) ^ li) << 4);

  // One tile pair (local tiles tl, tl+1) over row tiles a0 .. a0+NA-1 of the slot.
  auto pair_mma = [&]<int NA>(const uint8_t* sl, int tl, int a0, f32x4 (&ac)[NA][2]) __attribute__((always_inline)) {
    f16x8 wb[2][4];
    float dj[2][4];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint8_t* codes = sl + XB + (tl + b) * TB + lane * 16 * LB;
      const uint2 dd = *reinterpret_cast<const uint2*>(sl + XB + WB + (tl + b) * 128 + li * 8);
      uint4 v[LB];
#pragma unroll
      for (int c = 0; c < LB; ++c) v[c] = *reinterpret_cast<const uint4*>(codes + 16 * c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (layout_fmt(FMT) == CIR_Q4_0) {
          wb[b][j] = dq_q4((j == 0) ? v[0].x : (j == 1) ? v[0].y : (j == 2) ? v[0].z : v[0].w);
        } else {
          const uint4 vv = v[j >> 1];
          wb[b][j] = dq_q8((j & 1) ? vv.z : vv.x, (j & 1) ? vv.w : vv.y);
        }
        const uint32_t dw = (j < 2) ? dd.x : dd.y;
        dj[b][j] = static_cast<float>(__builtin_bit_cast(f16, (uint16_t)((j & 1) ? (dw >> 16) : (dw & 0xFFFFu))));
      }
    }
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      f16x8 xf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) xf[j] = *reinterpret_cast<const f16x8*>(sl + (a0 + a) * 4096 + xo[j]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x4 c[2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
          c[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wb[b][j], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) ac[a][b][r] = fmaf(dj[b][j], c[b][r], ac[a][b][r]);
      }
    }
  };
  auto compute = [&](const uint8_t* sl) __attribute__((always_inline)) {
    if (own) pair_mma.template operator()<MT>(sl, 2 * wave, 0, acc);
    if (fifth) pair_mma.template operator()<MT5>(sl, 2 * (kXwPairs - 1), wave * MT5, acc5);
  };

  // Quad i computes from slot i & 1 while quad i+1 comes into the other; the wait for
  // that DMA and the barrier end the step.
  xw_dma<FMT, MT, W>(slot_a, rx, rw, rd, xoff, wave, lane, t0, ntl, KQ, q0);
  __syncthreads();
  int i = 0;
#pragma nounroll
  for (; i + 2 <= nqs; i += 2) {
    if (i + 1 < nqs) xw_dma<FMT, MT, W>(slot_b, rx, rw, rd, xoff, wave, lane, t0, ntl, KQ, q0 + i + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(slot_a);
    __syncthreads();
    if (i + 2 < nqs) xw_dma<FMT, MT, W>(slot_a, rx, rw, rd, xoff, wave, lane, t0, ntl, KQ, q0 + i + 2);
    __builtin_amdgcn_sched_barrier(0);
    compute(slot_b);
    __syncthreads();
  }
  if (i < nqs) compute(slot_a);  // an odd count: the last quad sits in slot a
  if constexpr (kAccScale<FMT> != 1.f) {
#pragma unroll
    for (int a = 0; a < MT; ++a) acc[a][0] *= kAccScale<FMT>, acc[a][1] *= kAccScale<FMT>;
#pragma unroll
    for (int a = 0; a < MT5; ++a) acc5[a][0] *= kAccScale<FMT>, acc5[a][1] *= kAccScale<FMT>;
  }

  // SwiGLU of pair p of the run (gate tile t0 + 2p, up tile t0 + 2p + 1) over row tiles a0 .. a0+NA-1.
  auto store = [&]<int NA>(int p, int a0, const f32x4 (&ac)[NA][2]) __attribute__((always_inline)) {
    const int nt = t0 + 2 * p;
    const int inter = N / 2;
    const int col = (nt >> 1) * 16 + li;
    if (nt + 1 < NTILES && col < inter) {
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * (a0 + a) + 4 * lg + r;
          const float g = ac[a][0][r], u = ac[a][1][r];
          if (m < M) act[(size_t)m * inter + col] = static_cast<TO>(as_f32_value((g / (1.0f + expf(-g))) * u));
        }
    }
  };
  if (own) store.template operator()<MT>(wave, 0, acc);
  if (fifth) store.template operator()<MT5>(kXwPairs - 1, wave * MT5, acc5);
}

// m <= 8 (qgemv_kernel): a workgroup of W wavefronts owns W*NT row tiles, and each
// wavefront streams its own NT tiles over the workgroup's k-range (grid.y splits k)
// with no barrier inside the loop.  The m activation rows of that k-range are staged
// in LDS once, at the start, while the first weight stages are already in flight;
// per column that is 2*m bytes of activations against 9*W*NT bytes of weights.
// The MFMA is the GEMM's 16x16x32 step with activation rows past m repeating row
// m-1 (those outputs are never stored); only the MR accumulator registers that hold
// rows < m (rows 4*lg + r, r < MR) are scaled and kept.
constexpr int kGemvMaxRowQuads = 256;  // m * quads per split; LDS = m * 256 * quads B (<= 64 KiB)
constexpr int kGemvMaxWaves = 16;

// Workgroup = blockDim.x / 64 wavefronts (runtime); wavefront v of workgroup g in
// split s owns tiles (g * W + v) * tpw .. + tpw - 1 and streams them one after the
// other, each over the split's nq quads: tpw * nq ring stages with no drain between
// tiles.  A finished tile's accumulators go to the epilogue and restart at zero.
// XC: 16-byte activation chunks per thread (the host makes XC * blockDim.x cover
// the m * 16 * nq chunks of the split).
// EPI 0: fp32 split-k partials part[s][m][n].
// EPI 2 (one split): greedy head; each wavefront writes, per row, the best
//   (value, column) of its tiles to cand_v / cand_i [m][wavefront] (part and out),
//   for argmax_cand_kernel; TW = wavefronts that own tiles.
// (The fused SwiGLU stays on the GEMM kernel at every m: gate/up tiles must be
// consumed in pairs, and no GEMV geometry of pairs beat the GEMM's two-tile stages,
// 21.4 us against 19.2 at m = 1 for the Llama-3-8B gate|up.)
// Split decode-attention partials as a GEMV input (XM): per (row, head) S <= 8 partial
// outputs O_s [128] and (max, sum) pairs, laid out as the attention kernel writes them.
struct AttnParts {
  const float* o;   // [rows][heads][S][128]
  const float* ml;  // [rows][heads][S][2]
  int S, heads;
};
constexpr int kAttnMaxParts = 8;

// 8 consecutive head dims (d0..d0+7) of one (row, head) of the merged attention output,
// rounded to fp16 with the arithmetic and order of attn_merge (attention.hip): the same
// fmaf chains and o * inv rounded to fp32 before the fp16 conversion in both (left to
// itself the compiler fuses one of them into a single-rounding v_fma_mixlo_f16, which
// put one value in ~16k one fp16 ulp apart), so both paths give the same bits.
// All loads are issued first.
__device__ __forceinline__ u32x4 attn_merged_chunk(const AttnParts& a, int row, int head, int d0) {
  const float* ml = a.ml + ((size_t)row * a.heads + head) * a.S * 2;
  const float* po = a.o + ((size_t)row * a.heads + head) * a.S * 128 + d0;
  float2 mv[kAttnMaxParts];
  float4 o0[kAttnMaxParts], o1[kAttnMaxParts];
#pragma unroll
  for (int s = 0; s < kAttnMaxParts; ++s) {
    const int ss = s < a.S ? s : 0;
    mv[s] = *reinterpret_cast<const float2*>(ml + 2 * ss);
    o0[s] = *reinterpret_cast<const float4*>(po + (size_t)ss * 128);
    o1[s] = *reinterpret_cast<const float4*>(po + (size_t)ss * 128 + 4);
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < kAttnMaxParts; ++s)
    if (s < a.S) M = fmaxf(M, mv[s].x);
  float w[kAttnMaxParts];
#pragma unroll
  for (int s = 0; s < kAttnMaxParts; ++s) w[s] = (s < a.S && M != -INFINITY) ? exp2f(mv[s].x - M) : 0.f;
  float den = 0.f;
  if (M != -INFINITY)
#pragma unroll
    for (int s = 0; s < kAttnMaxParts; ++s)
      if (s < a.S) den = fmaf(mv[s].y, w[s], den);
  const float inv = den > 0.f ? 1.f / den : 0.f;
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kAttnMaxParts; ++s)
    if (s < a.S) {
      const float v[8] = {o0[s].x, o0[s].y, o0[s].z, o0[s].w, o1[s].x, o1[s].y, o1[s].z, o1[s].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = fmaf(v[e], w[s], o[e]);
    }
  uint32_t h[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const f16x2 two = {static_cast<f16>(as_f32_value(o[2 * e] * inv)), static_cast<f16>(as_f32_value(o[2 * e + 1] * inv))};
    h[e] = __builtin_bit_cast(uint32_t, two);
  }
  return u32x4{h[0], h[1], h[2], h[3]};
}

template <int FMT, int MR, int DW, int XC, int EPI = 0, typename TO = float, bool XM = false>
__global__ __launch_bounds__(64 * kGemvMaxWaves) void qgemv_kernel(const f16* __restrict__ x, int ldx,
                                                                 const uint8_t* __restrict__ wq,
                                                                 const uint16_t* __restrict__ wd,
                                                                 float* __restrict__ part, int M, int N, int K,
                                                                 int nq, int tpw, TO* __restrict__ out = nullptr,
                                                                 int TW = 0, AttnParts ap = AttnParts{}) {
  static_assert(EPI == 0 || EPI == 2, "GEMV epilogues: partials or argmax candidates");
  static_assert(!XM || (EPI == 0 && !is_row_fmt(FMT)), "attention-partials input: block formats, partials out");
  static_assert(EPI == 0 || !is_row_fmt(FMT), "row formats scale after the loop: EPI 0 only");
  constexpr int LB = Stage<FMT, 1, 1>::LB;
  extern __shared__ __align__(16) uint8_t xs[];
  const int W = __builtin_amdgcn_readfirstlane(blockDim.x >> 6);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, li = lane & 15, lg = lane >> 4;
  const int KQ = K / 128, NTILES = (N + 15) / 16;
  const int t0 = (blockIdx.x * W + wave) * tpw;  // this wavefront's first tile
  const int split = blockIdx.y;
  const int q0 = split * nq;
  // LDS: row r of the split's activations at r * 256 nq; its 16-byte chunk c sits in
  // slot c ^ (r & 7) of its 8-chunk group, so the fragment reads of rows 0..7 (same
  // chunk c) land in 8 different bank groups.
  const int rs = 256 * nq;

  // Activation loads first (the load counter retires in order, so the LDS writes
  // below wait for these and not for the weight stages issued after them).
  // Chunk c (16 B) = row c / (16 nq), column chunk c % (16 nq); chunks past the end
  // repeat the last one (same value to the same LDS address).
  const int nthr = 64 * W;
  const int cols16 = 16 * nq;
  const int r_step = nthr / cols16, c_step = nthr - r_step * cols16;  // uniform
  u32x4 xv[XC];
  int xoff[XC];
  {
    int r = (int)threadIdx.x / cols16, col = (int)threadIdx.x - r * cols16;
#pragma unroll
    for (int u = 0; u < XC; ++u) {
      const bool past = r >= M;
      const int rr = past ? M - 1 : r, cc = past ? cols16 - 1 : col;
      xoff[u] = rr * rs + 16 * (cc ^ (rr & 7));
      if constexpr (XM) {  // quad q of k is head q (head_dim 128)
        // The merge has waited for its loads already: its chunk goes to LDS at once rather
        // than staying live across the weight prologue (eight such chunks per thread spill).
        *reinterpret_cast<u32x4*>(&xs[xoff[u]]) = attn_merged_chunk(ap, rr, q0 + (cc >> 4), 8 * (cc & 15));
      } else {
        xv[u] = *reinterpret_cast<const u32x4*>(x + (size_t)rr * ldx + 128 * q0 + 8 * cc);
      }
      r += r_step;
      col += c_step;
      if (col >= cols16) col -= cols16, ++r;
    }
  }

  // Weight loads go through buffer resources: the tile offset is wavefront-uniform
  // (an SGPR), the lane offset a fixed VGPR, so no 64-bit address lives in VGPRs.
  const uint32_t ntiles_total = (uint32_t)NTILES * KQ;
  const rsrc_t rw = make_rsrc(wq, ntiles_total * 1024u * LB);
  const rsrc_t rd = make_rsrc(wd, is_row_fmt(FMT) ? 0u : ntiles_total * 128u);
  const uint32_t vw = (uint32_t)lane * 16u * LB, vd = (uint32_t)li * 8u;
  struct WS {
    uint4 w[LB];
    uint2 d;
  };
  // Ring of DW + 1 slots: the stage of quad i loads stage i + DW into the slot that
  // stage i - 1 has just freed, so no slot holds two live values and the loads go out
  // before the stage's compute.
  constexpr int R = DW + 1;
  WS ws[R];
  int il = 0, iq = 0;  // next stage to load: tile il of the wavefront, quad iq of the split
  auto issue = [&](int slot) __attribute__((always_inline)) {  // past the last stage: reload the last
    const bool past = il >= tpw;
    const uint32_t tb = (uint32_t)min(t0 + (past ? tpw - 1 : il), NTILES - 1) * KQ + q0 + (past ? nq - 1 : iq);
#pragma unroll
    for (int c = 0; c < LB; ++c) ws[slot].w[c] = buf16(rw, vw + 16u * c, tb * 1024u * LB);
    if constexpr (!is_row_fmt(FMT)) ws[slot].d = buf8(rd, vd, tb * 128u);
    if (++iq == nq) iq = 0, ++il;
  };
  auto each = [&]<int C>(auto&& f) __attribute__((always_inline)) {
    [&]<int... S>(std::integer_sequence<int, S...>) { (f.template operator()<S>(), ...); }(
        std::make_integer_sequence<int, C>{});
  };
  each.template operator()<DW>([&]<int S>() { issue(S); });

  if constexpr (!XM) {
#pragma unroll
    for (int u = 0; u < XC; ++u) *reinterpret_cast<u32x4*>(&xs[xoff[u]]) = xv[u];
  }
  __syncthreads();

  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  f32x4 sx = {0.f, 0.f, 0.f, 0.f};  // row formats: activation sums of this split
  const int xr = min(li, M - 1);
  const uint8_t* xrow = xs + xr * rs;
  int xo[4];  // swizzled byte offset of chunk 4j + lg inside a quad
#pragma unroll
  for (int j = 0; j < 4; ++j) xo[j] = ((4 * j + lg) ^ (xr & 7)) << 4;
  int cl = 0, cq = 0;  // stage being computed
  float bv[MR];  // EPI 2: best (value, column) per row
  int bi[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) bv[r] = -INFINITY, bi[r] = 0x7fffffff;

  // Rows past m hold MFMA results nobody reads; acc rows are 4 * lg + r.
  auto store_tile = [&]() __attribute__((always_inline)) {
    const int t = t0 + cl;
    const int n = t * 16 + li;
    if constexpr (kAccScale<FMT> != 1.f) {
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r] *= kAccScale<FMT>;
    }
    if constexpr (is_row_fmt(FMT)) {
      // w = (c - zp) * s with c the stored code: acc holds sum x*c over this split,
      // so the split's share of y is s * (acc + (c0 - zp) * sum x), c0 - zp = offset[row].
      const float* rscale = reinterpret_cast<const float*>(wd);
      const float* roff = rscale + (size_t)NTILES * 16;
      const int nn = min(t, NTILES - 1) * 16 + li;
      const float sc = rscale[nn], of = roff[nn];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r] = sc * fmaf(of, sx[r], acc[r]);
    }
    if constexpr (EPI == 2) {
      if (t < NTILES && n < N) {
#pragma unroll
        for (int r = 0; r < MR; ++r) argmax_better(bv[r], bi[r], acc[r], n);
      }
    } else {
      if (t < NTILES && n < N) {
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const int m = 4 * lg + r;
          if (m < M) part[((size_t)split * M + m) * N + n] = acc[r];
        }
      }
    }
    acc = f32x4{0.f, 0.f, 0.f, 0.f};
    sx = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  auto compute = [&](const WS& st) __attribute__((always_inline)) {
    f16x8 xf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xf[j] = *reinterpret_cast<const f16x8*>(xrow + 256 * cq + xo[j]);
    auto wfr = [&](int j) __attribute__((always_inline)) {
      f16x8 wb;
      if constexpr (layout_fmt(FMT) == CIR_Q4_0) {
        const uint4 v = st.w[0];
        wb = dq_q4((j == 0) ? v.x : (j == 1) ? v.y : (j == 2) ? v.z : v.w);
      } else {
        const uint4 v = st.w[j >> 1];
        wb = dq_q8((j & 1) ? v.z : v.x, (j & 1) ? v.w : v.y);
      }
      return wb;
    };
    auto scale_of = [&](int j) __attribute__((always_inline)) {
      const uint32_t dw = (j < 2) ? st.d.x : st.d.y;
      return static_cast<float>(__builtin_bit_cast(f16, (uint16_t)((j & 1) ? (dw >> 16) : (dw & 0xFFFFu))));
    };
    if constexpr (is_row_fmt(FMT)) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f16x8 wb = wfr(j);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wb, acc, 0, 0, 0);
        const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
        sx = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], ones, sx, 0, 0, 0);
      }
    } else if constexpr (MR == 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wfr(j), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        acc[0] = fmaf(scale_of(j), c[0], acc[0]);
      }
    } else {
      // Several rows: block j+1's MFMA goes out before block j's scale FMAs (same arithmetic and order;
      // config 3's down at m = 8: 9.5-10.0 -> 9.4-9.7 us over two boxes; at m = 1 it measured no better)
      f32x4 c[4];
      auto mf = [&](int j) __attribute__((always_inline)) {
        c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[j], wfr(j), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      };
      auto fm = [&](int j) __attribute__((always_inline)) {
        const float dj = scale_of(j);
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[r] = fmaf(dj, c[j][r], acc[r]);
      };
      mf(0);
      mf(1);
      fm(0);
      mf(2);
      fm(1);
      mf(3);
      fm(2);
      fm(3);
    }
    if (cq == nq - 1) store_tile();  // uniform
    if (++cq == nq) cq = 0, ++cl;
  };

  const int T = tpw * nq;
  int i = 0;
#pragma nounroll
  for (; i + R <= T; i += R) {
    each.template operator()<R>([&]<int S>() {
      issue((S + DW) % R);
      compute(ws[S]);
      __builtin_amdgcn_sched_barrier(0);  // keep stages apart: hoisting across them only adds registers
    });
  }
  each.template operator()<DW>([&]<int S>() {  // at most DW stages are left, in slots 0 .. DW-1
    if (i + S < T) compute(ws[S]);
  });

  if constexpr (EPI == 2) {
    // the 16 lanes of a row group (same lg) hold 16 different columns
    float* cand_v = part;
    int* cand_i = reinterpret_cast<int*>(out);
    const int vg = blockIdx.x * W + wave;
#pragma unroll
    for (int r = 0; r < MR; ++r) {
#pragma unroll
      for (int off = 8; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv[r], off, 64);
        const int oi = __shfl_xor(bi[r], off, 64);
        argmax_better(bv[r], bi[r], ov, oi);
      }
      const int m = 4 * lg + r;
      if (li == 0 && m < M && vg < TW) {
        cand_v[(size_t)m * TW + vg] = bv[r];
        cand_i[(size_t)m * TW + vg] = bi[r];
      }
    }
  }
}

#ifndef CIR_GV_DW
#define CIR_GV_DW 4
#endif

bool gemv_fits(int m, int k, int splits) { return m <= 8 && m * ((k / 128) / splits) <= kGemvMaxRowQuads; }

// GEMV launch geometry for a given split: W wavefronts per workgroup and tpw tiles per
// wavefront.  Every workgroup should be resident at once and every CU should stream
// the same number of tile-quads, since a CU's share of HBM bandwidth is bounded (its
// L1 miss queue): the busiest CU sets the time.  Measured on MI355X at the Llama-3-8B
// shapes: 6-8 wavefronts per CU stream best (4 leave the miss queue short, 14-16
// lose 1-4 us), and the number of tiles per wavefront hardly matters.  So W is 6..8
// and, among those, take the least busiest-CU work, then the fewest workgroups (each
// stages its activations once).
struct GemvGeom {
  int waves, tpw;
};
constexpr int kCUs = 256;
// W also keeps the activation staging within 8 chunks per thread.
GemvGeom gemv_geometry(int m, int n, int k, int splits) {
  const int ntiles = (n + 15) / 16, nq = (k / 128) / splits;
  const size_t lds = (size_t)m * 256 * nq;
  GemvGeom best{8, 1};
  long best_work = -1, best_groups = 0;
  for (int w = 6; w <= 8; ++w) {
    if (16 * m * nq > 8 * 64 * w) continue;
    const int by_lds = (int)(160 * 1024 / lds);
    const int per_cu_cap = min(32 / w, by_lds);  // resident workgroups per CU (8 wavefronts per SIMD)
    if (per_cu_cap < 1) continue;
    for (int tpw = 1; tpw <= 64; ++tpw) {
      const long groups = (long)splits * ((ntiles + w * tpw - 1) / (w * tpw));
      const long per_cu = (groups + kCUs - 1) / kCUs;
      if (per_cu > per_cu_cap) continue;
      const long work = per_cu * w * tpw * nq;
      if (best_work < 0 || work < best_work || (work == best_work && groups < best_groups)) {
        best = GemvGeom{w, tpw};
        best_work = work;
        best_groups = groups;
      }
    }
  }
  return best;
}

// GEMV k-split: over powers of two with m * quads <= kGemvMaxRowQuads, the least
// estimated time: busiest-CU weight bytes at 7 TB/s / 256 plus the partials written
// and read back by the epilogue (8 * splits * m * n bytes at 7 TB/s).  0: none fits.
int gemv_splits(int m, int n, int k) {
  const int kq = k / 128;
  int best = 0;
  double best_t = 0;
  for (int s = 1; s <= kq && s <= 64; s *= 2) {
    if (kq % s || !gemv_fits(m, k, s)) continue;
    const GemvGeom g = gemv_geometry(m, n, k, s);
    const int ntiles = (n + 15) / 16, nq = kq / s;
    const long groups = (long)s * ((ntiles + g.waves * g.tpw - 1) / (g.waves * g.tpw));
    const long per_cu = (groups + kCUs - 1) / kCUs;
    const double t = per_cu * g.waves * g.tpw * nq * 1152.0 / (7e12 / kCUs) + 8.0 * s * m * n / 7e12;
    if (!best || t < best_t) best = s, best_t = t;
  }
  return best;
}

// One GEMV launch: EPI 0 (partials into part) or 2 (argmax candidates into part /
// out, one split).  Returns the number of wavefronts that own tiles (the candidate
// count per row for EPI 2).
template <int FMT, int EPI, typename TO = float, bool XM = false>
int launch_qgemv(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, float* part, int M, int N, int K,
                 int splits, hipStream_t s, TO* out = nullptr, AttnParts ap = AttnParts{}) {
  const int NTILES = (N + 15) / 16;
  const int nq = (K / 128) / splits;
  GemvGeom g = gemv_geometry(M, N, K, splits);
  if constexpr (is_row_fmt(FMT)) g.tpw = 1;  // the row scales are read once, after the loop
  const int waves_per_split = (NTILES + g.tpw - 1) / g.tpw;
  dim3 grid((waves_per_split + g.waves - 1) / g.waves, splits);
  const size_t lds = (size_t)M * 256 * nq;
  const int xc_need = (16 * M * nq + 64 * g.waves - 1) / (64 * g.waves);
  auto go = [&]<int MR, int XC>() {
    qgemv_kernel<FMT, MR, CIR_GV_DW, XC, EPI, TO, XM>
        <<<grid, 64 * g.waves, lds, s>>>(x, ldx, wq, wd, part, M, N, K, nq, g.tpw, out, waves_per_split, ap);
  };
  auto by_xc = [&]<int MR>() {
    if (xc_need <= 1) go.template operator()<MR, 1>();
    else if (xc_need <= 2) go.template operator()<MR, 2>();
    else if (xc_need <= 4) go.template operator()<MR, 4>();
    else go.template operator()<MR, 8>();
  };
  // Row formats keep all four accumulator rows: their MFMA chains carry every row to
  // the final scale, which reads them all (no row's registers are freed early).
  if constexpr (is_row_fmt(FMT)) {
    by_xc.template operator()<4>();
  } else {
    if (M == 1) by_xc.template operator()<1>();
    else if (M == 2) by_xc.template operator()<2>();
    else by_xc.template operator()<4>();
  }
  return waves_per_split;
}

// The greedy head takes the GEMV when m <= 8 and the whole k fits one split's
// activation stage (block formats only).
bool gemv_head_fits(int fmt, int m, int k) { return !is_row_fmt(fmt) && gemv_fits(m, k, 1); }

#ifndef CIR_XS_DW
#define CIR_XS_DW 4
#endif
#ifndef CIR_XS_DW_SWIGLU
#define CIR_XS_DW_SWIGLU 4
#endif
#ifndef CIR_XS_KG
#define CIR_XS_KG 1
#endif

// Weight-ring depth of the m <= 32 kernel: 8-bit codes (two 16-byte loads per lane and tile) at 32 rows take 3
// stages where the launch has two k-groups or the greedy epilogue; at 4 stages those need more than 256 VGPRs
// and spill.
template <int FMT, int MT, int EPI, int KG, int DW>
inline constexpr int xs_ring = (layout_fmt(FMT) == CIR_Q8_0 && MT >= 2 && (KG >= 2 || EPI == 2) && DW > 3) ? 3 : DW;

// k-groups per workgroup: a divisor of the split's quad count.  Two where a split has
// 32 quads or more and the launch has at most one workgroup per CU, at any m
// (measured: the unsplit gate|up + SwiGLU at k = 4096, 224 workgroups, gains ~4% at
// m = 32 and ~10% at m = 1; the lm_head's 1002 workgroups lose 15%, and splits of
// 4-14 quads lose with half as many per group).  The count depends on the launch's
// workgroup count, which differs between epilogues: at m <= 16 the partials launch
// (NT = 1) can have twice the workgroups of the SwiGLU launch (NT = 2) and take one
// group where the SwiGLU takes two, so there the two sum the quads in different orders
// and agree to rounding, not bit for bit.
int xs_kgroups(int m, int quads, long workgroups) {
  int kg = (quads >= 32 && workgroups <= kCUs) ? 2 : (m > 16 ? CIR_XS_KG : 1);
  while (kg > 1 && quads % kg) kg /= 2;
  return kg;
}

template <int FMT, int MT, typename TO>
void launch_qgemm_swiglu(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, TO* act, int M, int N, int K,
                         hipStream_t s) {
  const int NTILES = (N + 15) / 16;
  dim3 grid((NTILES + 7) / 8, 1, (M + 16 * MT - 1) / (16 * MT));
  // One row (batch 1) scales only accumulator row 0 (MR = 1): gate|up + SwiGLU at the Llama-3-8B shape 16.9-17.7
  // -> 16.1-16.6 us isolated, batch-1 step 1.741-1.743 -> 1.738-1.740 ms (three alternated pairs); the same bits.
  auto go = [&]<int KG>() {
    if (M == 1)
      qgemm_xs_kernel<FMT, 2, MT, xs_ring<FMT, MT, 1, KG, CIR_XS_DW_SWIGLU>, 1, TO, KG, 1>
          <<<grid, 256 * KG, 0, s>>>(x, ldx, wq, wd, nullptr, M, N, K, K / 128, act);
    else
      qgemm_xs_kernel<FMT, 2, MT, xs_ring<FMT, MT, 1, KG, CIR_XS_DW_SWIGLU>, 1, TO, KG>
          <<<grid, 256 * KG, 0, s>>>(x, ldx, wq, wd, nullptr, M, N, K, K / 128, act);
  };
  const int kg = xs_kgroups(M, K / 128, (long)grid.x * grid.y * grid.z);
  if constexpr (CIR_XS_KG >= 4) {
    if (kg == 4) return go.template operator()<4>();
  }
  if (kg == 2) go.template operator()<2>();
  else go.template operator()<1>();
}

// ids[m] = best candidate of row m over the W wavefront candidates (any order: the
// candidates carry their columns, so ties resolve to the smallest column).
__global__ __launch_bounds__(256) void argmax_cand_kernel(const float* __restrict__ cand_v, const int* __restrict__ cand_i,
                                                          int W, int M, int64_t* __restrict__ ids) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int m = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const float* cv = cand_v + (size_t)m * W;
  const int* ci = cand_i + (size_t)m * W;
  // 8 candidates per thread in flight at a time: the loop is latency-bound otherwise
  // (one L2 round trip per candidate; 4008 per row for a 128256-column head).
  constexpr int U = 8;
  for (int w0 = threadIdx.x; w0 < W; w0 += 256 * U) {
    float v[U];
    int ix[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int w = w0 + 256 * u;
      v[u] = w < W ? cv[w] : -INFINITY;
      ix[u] = w < W ? ci[w] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) argmax_better(bv, bi, v[u], ix[u]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    argmax_better(bv, bi, ov, oi);
  }
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = bv;
    si[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w) argmax_better(bv, bi, sv[w], si[w]);
    ids[m] = bi == 0x7fffffff ? 0 : bi;
  }
}

// Wavefront candidates of the fused head: one per 64*NT columns and row.
constexpr int xs_rows_per_wave(int m) { return m <= 16 ? 16 : 32; }
size_t argmax_cand_count(int m, int n) {
  const int rows_per_group = 4 * xs_rows_per_wave(m);
  return (size_t)((n + rows_per_group - 1) / rows_per_group) * 4 * m;
}

template <int FMT, int NT, int MT>
void launch_qgemm_argmax(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, float* cand_v, int* cand_i,
                         int64_t* ids, int M, int N, int K, hipStream_t s) {
  const int NTILES = (N + 15) / 16;
  dim3 grid((NTILES + 4 * NT - 1) / (4 * NT), 1, (M + 16 * MT - 1) / (16 * MT));
  const int quads = K / 128;
  auto go = [&]<int KG>() {
    qgemm_xs_kernel<FMT, NT, MT, xs_ring<FMT, MT, 2, KG, (MT == 1 ? 4 : CIR_XS_DW)>, 2, float, KG>
        <<<grid, 256 * KG, 0, s>>>(x, ldx, wq, wd, cand_v, M, N, K, quads, reinterpret_cast<float*>(cand_i));
  };
  const int kg = xs_kgroups(M, quads, (long)grid.x * grid.y * grid.z);
  if constexpr (CIR_XS_KG >= 4) {
    if (kg == 4) return go.template operator()<4>(), argmax_cand_kernel<<<M, 256, 0, s>>>(cand_v, cand_i, (int)grid.x * 4, M, ids);
  }
  if (kg == 2) go.template operator()<2>();
  else go.template operator()<1>();
  argmax_cand_kernel<<<M, 256, 0, s>>>(cand_v, cand_i, (int)grid.x * 4, M, ids);
}

template <int FMT, int NT, int MT, int DW>
void launch_qgemm_xs(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, float* part, int M, int N, int K,
                     int splits, hipStream_t s) {
  const int NTILES = (N + 15) / 16;
  dim3 grid((NTILES + 4 * NT - 1) / (4 * NT), splits, (M + 16 * MT - 1) / (16 * MT));
  const int quads = (K / 128) / splits;
  auto go = [&]<int KG>() {
    qgemm_xs_kernel<FMT, NT, MT, xs_ring<FMT, MT, 0, KG, DW>, 0, float, KG>
        <<<grid, 256 * KG, 0, s>>>(x, ldx, wq, wd, part, M, N, K, quads);
  };
  const int kg = xs_kgroups(M, quads, (long)grid.x * grid.y * grid.z);
  if constexpr (CIR_XS_KG >= 4) {
    if (kg == 4) return go.template operator()<4>();
  }
  if (kg == 2) go.template operator()<2>();
  else go.template operator()<1>();
}

// Large m: activation rows per workgroup (16 * MT).
constexpr int xl_mt(int m) { return m <= 64 ? 4 : 8; }
// The large-m SwiGLU launch (one split, so the column groups alone set the workgroup
// count; at 32 < m <= 128 it serves the row formats, which the balanced kernel does not
// take) keeps 64 rows per workgroup up to m = 128: at the Qwen2-7B gate|up (n 37888, 296
// column groups) 128 rows per workgroup leave 296 workgroups, a second round on 40 CUs,
// while two 64-row blocks give 592 smaller ones at 3 wavefronts per SIMD (158 VGPRs
// against 202): 83.2-86.0 us against 90.3-90.9 (Q8_0, m = 128, same box, alternated).
// The partials launch keeps xl_mt (QKV, n 4608: 19.3 us at 64 rows against 16.4).
constexpr int xl_mt_swiglu(int m) { return m <= 128 ? 4 : 8; }

// Workgroups of the large-m kernel before any k-split: groups of 128 columns x blocks of 16*MT rows.
long xl_groups(int m, int n) { return (long)((n + 127) / 128) * ((m + 16 * xl_mt(m) - 1) / (16 * xl_mt(m))); }

// m > 32 takes the large-m kernel when n spans at least 36 groups of 128 columns, when
// its workgroups alone fill the CUs (>= 192: large m), or, where k may be split, when k
// holds at least 64 quads (the k-split pieces then stay long).  Measured at the Qwen2-7B
// shapes (Q8_0, m = 64 / 128) against the m <= 32 kernel run over 32-row blocks: QKV
// (n 4608) 11.0 / 16.9 us against 15.4 / 24.5, gate|up (n 37888) 51.6 / 81.8 against
// 72.6 / 114.9; down (n 3584, 28 groups, k 18944) at m = 128: 42.3 us over 9 splits
// against 49.1 / 66.4 for the small kernel at 4 / 2 splits; O (n 3584, k 3584: 28 quads)
// stays on the small kernel (12.4-12.7 us against 14.6 at 7 splits).  At m = 2048
// (Llama-3-8B, Q4_0) the large kernel takes down 353.8 -> 287.8 us and O 113.8 -> 95.2.
// The SwiGLU launch cannot split k (splittable = false).
bool use_xl(int m, int n, int k, bool splittable = true) {
  if (m <= 32) return false;
  return (n + 127) / 128 >= 36 || xl_groups(m, n) >= 192 || (splittable && k / 128 >= 64);
}

// Its k-split: as many splits as keep the launch at one round of workgroups over the
// 256 CUs (down at m = 128: 9 splits, 252 workgroups: 42.3 us against 46.5 at 8 and 43.9
// at 10), each split at least 4 quads.  The splits need not divide k/128: split s covers
// quads s * ceil(kq / S) onward, the last one fewer.  The count is then lowered to
// ceil(kq / len) for that split length len, so the last split is never empty (86 quads
// at 16 splits would leave split 15 starting past the end; 15 splits of 6 quads do not).
int xl_splits(int m, int n, int k) {
  const long kq = k / 128;
  const long by_cus = 256 / xl_groups(m, n), by_len = kq / 4;
  long s = by_cus < by_len ? by_cus : by_len;
  if (s <= 1) return 1;
  const long len = (kq + s - 1) / s;
  s = (kq + len - 1) / len;
  return (int)s;
}

// The k-splits a cir_qgemm launch accepts: those dividing k/128, and on the large-m
// kernel any count whose every split holds at least one quad.
bool splits_ok(int m, int n, int k, int splits) {
  const int kq = k / 128;
  if (splits < 1 || splits > kq) return false;
  if (kq % splits == 0) return true;
  return use_xl(m, n, k) && (splits - 1) * ((kq + splits - 1) / splits) < kq;
}

#ifndef CIR_XL_W
#define CIR_XL_W 4
#endif
template <int FMT, int MT, int EPI, typename TO = float>
void launch_qgemm_xl(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, float* part, int M, int N, int K,
                     int splits, hipStream_t s, TO* act = nullptr) {
  // Ring of DW + 1 = 4 weight stages for both widths: an even ring lets the activation
  // DMA go out before the compute (the kernel's even-ring path).  Q4_0 at m = 2048 (a
  // 2048-token prefill): down 301-303 -> 289.9-290.3 us, QKV 147.8-148.2 -> 138.9-140.0
  // against a 5-stage ring, prefill 46.7-46.8 -> 44.2 ms (6 stages: 44.4-44.7).
  constexpr int DW = 3;
  constexpr int W = CIR_XL_W;
  const int NTILES = (N + 15) / 16;
  dim3 grid((NTILES + 2 * W - 1) / (2 * W), splits, (M + 16 * MT - 1) / (16 * MT));
  const int nq = (K / 128 + splits - 1) / splits;
  // Q8_0 partials in one round of workgroups (decode at m <= 128) take the interleave hint: at config 5 (m = 128)
  // QKV 15.7 -> 14.6-14.8 us, down 41.7 -> 38.8-39.0.  Where the workgroups outnumber the CUs (prefill) its extra
  // registers cost occupancy (Q8_0 m = 2048: QKV 120.3 -> 130.8 us), and Q4_0's lighter dequant gains nothing.
  if constexpr (FMT == CIR_Q8_0 && EPI == 0) {
    if ((long)grid.x * grid.y * grid.z <= kCUs) {
      qgemm_xl_kernel<FMT, MT, DW, EPI, TO, W, true><<<grid, 64 * W, 0, s>>>(x, ldx, wq, wd, part, M, N, K, nq, act);
      return;
    }
  }
  // Launches of more workgroups than CUs (prefill sizes) convert the scales once (PF): at m = 2048 (Q4_0) gate|up +
  // SwiGLU 568 -> 536 us, QKV 150 -> 142, O 98 -> 94, down 288 -> 282; a 2048-token prefill 43.7 -> 42.2 ms.
  // Together with the interleave hint it measured slower (config 5's Q8_0 QKV 14.3 -> 16.2 us), and in the
  // m <= 32 kernel and the GEMV too (batch-1 step 1.749 -> 1.771 ms).
  if constexpr (!is_row_fmt(FMT)) {
    if ((long)grid.x * grid.y * grid.z > kCUs) {
      qgemm_xl_kernel<FMT, MT, DW, EPI, TO, W, false, true><<<grid, 64 * W, 0, s>>>(x, ldx, wq, wd, part, M, N, K, nq, act);
      return;
    }
  }
  qgemm_xl_kernel<FMT, MT, DW, EPI, TO, W><<<grid, 64 * W, 0, s>>>(x, ldx, wq, wd, part, M, N, K, nq, act);
}

// The fused greedy head on the large-m kernel (one split): 128 columns per workgroup, one
// candidate per wavefront and row, as many as argmax_cand_count gives the m > 16 kernel.
// At the Qwen2-7B head (n 152064, k 3584, Q8_0) it reads the weights once per 16*MT rows
// where the m <= 32 kernel reads them once per 32: 495.6 us at m = 128 for the latter
// against 268.6 us for the large-m kernel's logits alone.
template <int FMT, int MT>
void launch_qgemm_xl_argmax(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, float* cand_v, int* cand_i,
                            int64_t* ids, int M, int N, int K, hipStream_t s) {
  constexpr int DW = 3;  // as in launch_qgemm_xl
  constexpr int W = CIR_XL_W;
  static_assert(2 * 16 * W == 128, "argmax_cand_count assumes 128 columns per workgroup");
  const int NTILES = (N + 15) / 16;
  dim3 grid((NTILES + 2 * W - 1) / (2 * W), 1, (M + 16 * MT - 1) / (16 * MT));
  qgemm_xl_kernel<FMT, MT, DW, 2, float, W>
      <<<grid, 64 * W, 0, s>>>(x, ldx, wq, wd, cand_v, M, N, K, K / 128, reinterpret_cast<float*>(cand_i));
  argmax_cand_kernel<<<M, 256, 0, s>>>(cand_v, cand_i, (int)grid.x * W, M, ids);
}

// The balanced large-m kernel's workgroups: one per CU while the tile pairs allow
// (1..5 pairs each), more only when the pairs exceed 5 per CU.
int xw_workgroups(int n) {
  const int np = ((n + 15) / 16 + 1) / 2;
  const int need = (np + kXwPairs - 1) / kXwPairs;
  const int one_round = np < kCUs ? np : kCUs;
  return need > one_round ? need : one_round;
}

// The fused SwiGLU at 32 < m <= 128 (block formats) runs the balanced kernel, 4 wavefronts
// (8, two per pair, measured no faster).  At the Qwen2-7B gate|up (Q8_0, 12 weight copies
// rotated): m = 128 78.6-81.0 us against 81.4-85.5 for the large-m kernel in 64-row
// blocks (64-row blocks of the balanced kernel: 84.9), m = 64 49.2-51.0 against 54.5-56.4.
// The gain is less than the per-CU bytes suggest (1.5 MB against 2.8 MB on the busiest
// CU): with one workgroup per CU the quads' DMA and compute alternate more than overlap.
bool use_xw_swiglu(int m) { return m > 32 && m <= 128; }

template <int FMT, int MT, typename TO>
void launch_qgemm_xw_swiglu(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, TO* act, int M, int N, int K,
                            hipStream_t s) {
  dim3 grid(xw_workgroups(N), 1, (M + 16 * MT - 1) / (16 * MT));
  qgemm_xw_kernel<FMT, MT, TO><<<grid, 64 * kXwWaves, 0, s>>>(x, ldx, wq, wd, M, N, K, act);
}

// Workgroup rows: 4 wavefronts x NT tiles x 16.  m <= 16 takes NT = 1 (64 rows per
// workgroup, MT = 1); larger m takes NT = 2, MT = 2 (128 rows x 32 activation rows):
// each activation quad then feeds 8 weight tiles.  Measured on MI355X at the
// Llama-3-8B shapes (m = 1, 8, 32) against NT = 4 and ring depths 2..6.
constexpr int xs_rows_per_group(int m) { return m <= 16 ? 64 : 128; }

// k-split: the smallest power of two that gives >= 192 workgroups, keeping at least
// 4 quads per split (split-k partials cost 4*m*n bytes each, so no more than needed).
// The threshold, swept on the config-4 step at m = 32 (same box, two passes each):
// 96 / 128 / 192 / 256 / 384 gave 3.80 / 3.69 / 3.45-3.54 / 3.58 / 3.70 ms.
int default_splits(int m, int n, int k) {
  if (m <= 8) {
    if (const int s = gemv_splits(m, n, k)) return s;
  }
  if (use_xl(m, n, k)) return xl_splits(m, n, k);
  const int kq = k / 128;
  const long groups = (long)((n + xs_rows_per_group(m) - 1) / xs_rows_per_group(m)) * ((m + 31) / 32);
  int s = 1;
  while (groups * s < 192 && kq % (2 * s) == 0 && kq / (2 * s) >= 4) s *= 2;
  return s;
}

template <int FMT>
void dispatch_qgemm(const f16* x, int ldx, const uint8_t* wq, const uint16_t* wd, float* part, int M, int N, int K,
                    int splits, hipStream_t s) {
  if (gemv_fits(M, K, splits)) launch_qgemv<FMT, 0>(x, ldx, wq, wd, part, M, N, K, splits, s);
  else if (M <= 16) launch_qgemm_xs<FMT, 1, 1, 4>(x, ldx, wq, wd, part, M, N, K, splits, s);
  else if (!use_xl(M, N, K)) launch_qgemm_xs<FMT, 2, 2, CIR_XS_DW>(x, ldx, wq, wd, part, M, N, K, splits, s);
  else if (M <= 64) launch_qgemm_xl<FMT, 4, 0>(x, ldx, wq, wd, part, M, N, K, splits, s);
  else launch_qgemm_xl<FMT, 8, 0>(x, ldx, wq, wd, part, M, N, K, splits, s);
}

}  // namespace
}  // namespace cir

using namespace cir;

extern "C" size_t cir_qweight_tiled_bytes(int fmt, int n, int k) {
  if (!valid_fmt(fmt) || n <= 0 || k <= 0 || k % 128) return 0;
  const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
  if (is_row_fmt(fmt)) return tiles * 64 * quant_bytes_per_lane(fmt) + (size_t)((n + 15) / 16) * 16 * 2 * sizeof(float);
  return tiles * (64 * quant_bytes_per_lane(fmt) + 16 * 4 * sizeof(uint16_t));
}

extern "C" int cir_qweight_repack_rows(const void* packed, const float* scales, const int32_t* zero_points, void* tiled,
                                       int fmt, int n, int k, void* stream) {
  CIR_CHECK_ARG(is_row_fmt(fmt), "repack_rows: fmt must be CIR_I4_ROW or CIR_I8_ROW (got %d)", fmt);
  CIR_CHECK_ARG(n >= 0 && k >= 0 && k % 128 == 0, "repack_rows: k (%d) must be a multiple of 128", k);
  if (n == 0 || k == 0) return 0;
  CIR_CHECK_ARG(packed && scales && zero_points && tiled, "repack_rows: null pointer");
  const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
  uint8_t* q = static_cast<uint8_t*>(tiled);
  float* rows = reinterpret_cast<float*>(q + tiles * 64 * quant_bytes_per_lane(fmt));
  const long threads = (long)tiles * 64;
  repack_rows_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, as_stream(stream)>>>(
      static_cast<const uint8_t*>(packed), scales, zero_points, q, rows, fmt, n, k);
  return launch_status();
}

extern "C" int cir_qweight_repack(const void* gguf_blocks, void* tiled, int fmt, int n, int k, void* stream) {
  CIR_CHECK_ARG(fmt == CIR_Q4_0 || fmt == CIR_Q8_0, "repack: fmt must be CIR_Q4_0 or CIR_Q8_0 (got %d)", fmt);
  CIR_CHECK_ARG(n >= 0 && k >= 0 && k % 128 == 0, "repack: k (%d) must be a multiple of 128", k);
  if (n == 0 || k == 0) return 0;
  CIR_CHECK_ARG(gguf_blocks && tiled, "repack: null pointer");
  const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
  uint8_t* q = static_cast<uint8_t*>(tiled);
  uint16_t* d = reinterpret_cast<uint16_t*>(q + tiles * 64 * quant_bytes_per_lane(fmt));
  const long threads = (long)tiles * 64;
  repack_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, as_stream(stream)>>>(static_cast<const uint8_t*>(gguf_blocks),
                                                                                 q, d, fmt, n, k);
  return launch_status();
}

extern "C" int cir_dequant(const void* weights, int tiled, int fmt, float* out, int n, int k, void* stream) {
  CIR_CHECK_ARG(valid_fmt(fmt), "dequant: unknown weight format %d", fmt);
  CIR_CHECK_ARG(tiled || !is_row_fmt(fmt), "dequant: row formats are read from their tiled copy (tiled = 1)");
  CIR_CHECK_ARG(n >= 0 && k >= 0 && k % 32 == 0, "dequant: k (%d) must be a multiple of 32", k);
  if (n == 0 || k == 0) return 0;
  CIR_CHECK_ARG(weights && out, "dequant: null pointer");
  hipStream_t s = as_stream(stream);
  if (!tiled) {
    const long nblk = (long)n * (k / 32);
    dequant_gguf_kernel<<<(unsigned)((nblk + 255) / 256), 256, 0, s>>>(static_cast<const uint8_t*>(weights), out, fmt,
                                                                      n, k);
  } else {
    CIR_CHECK_ARG(k % 128 == 0, "dequant: tiled weights need k %% 128 == 0");
    const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
    const uint8_t* q = static_cast<const uint8_t*>(weights);
    const void* d = q + tiles * 64 * quant_bytes_per_lane(fmt);
    const long threads = (long)tiles * 64;
    dequant_tiled_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(q, d, out, fmt, n, k);
  }
  return launch_status();
}

extern "C" int cir_qgemm_splits(int m, int n, int k) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 128) return 0;
  return cir::default_splits(m, n, k);
}

extern "C" size_t cir_qgemm_workspace_bytes(int m, int n, int splits) {
  if (m <= 0 || n <= 0 || splits <= 0) return 0;
  return (size_t)splits * m * n * sizeof(float);
}

extern "C" int cir_qgemm(const void* x, int ldx, const void* w_tiled, int fmt, float* y_partial, int m, int n, int k,
                         int splits, void* stream) {
  CIR_CHECK_ARG(valid_fmt(fmt), "qgemm: unknown weight format %d", fmt);
  CIR_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "qgemm: negative size");
  if (m == 0 || n == 0) return 0;
  CIR_CHECK_ARG(k > 0 && k % 128 == 0, "qgemm: k (%d) must be a positive multiple of 128", k);
  CIR_CHECK_ARG(splits_ok(m, n, k, splits),
                "qgemm: splits (%d) must divide k/128 (%d), or on the large-m kernel leave no split empty", splits,
                k / 128);
  CIR_CHECK_ARG(ldx >= k && ldx % 8 == 0, "qgemm: ldx (%d) must be >= k and a multiple of 8", ldx);
  CIR_CHECK_ARG(x && w_tiled && y_partial, "qgemm: null pointer");
  CIR_CHECK_ARG(splits <= 65535 && (m + 15) / 16 <= 65535, "qgemm: grid too large");
  const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
  const uint8_t* q = static_cast<const uint8_t*>(w_tiled);
  const uint16_t* d = reinterpret_cast<const uint16_t*>(q + tiles * 64 * quant_bytes_per_lane(fmt));
  const f16* xh = static_cast<const f16*>(x);
  hipStream_t s = as_stream(stream);
  if (fmt == CIR_Q4_0) {
    dispatch_qgemm<CIR_Q4_0>(xh, ldx, q, d, y_partial, m, n, k, splits, s);
  } else if (fmt == CIR_Q8_0) {
    dispatch_qgemm<CIR_Q8_0>(xh, ldx, q, d, y_partial, m, n, k, splits, s);
  } else if (fmt == CIR_I4_ROW) {
    dispatch_qgemm<CIR_I4_ROW>(xh, ldx, q, d, y_partial, m, n, k, splits, s);
  } else {
    dispatch_qgemm<CIR_I8_ROW>(xh, ldx, q, d, y_partial, m, n, k, splits, s);
  }
  return launch_status();
}

extern "C" int cir_qgemm_attn(const float* attn_part_o, const float* attn_part_ml, int attn_splits, int num_heads,
                              const void* w_tiled, int fmt, float* y_partial, int m, int n, int k, int splits,
                              void* stream) {
  CIR_CHECK_ARG(fmt == CIR_Q4_0 || fmt == CIR_Q8_0, "qgemm_attn: block formats only (got %d)", fmt);
  CIR_CHECK_ARG(m >= 0 && n >= 0 && num_heads > 0, "qgemm_attn: bad sizes");
  if (m == 0 || n == 0) return 0;
  CIR_CHECK_ARG(k == num_heads * 128, "qgemm_attn: k (%d) must be num_heads (%d) x 128", k, num_heads);
  CIR_CHECK_ARG(attn_splits >= 1 && attn_splits <= cir::kAttnMaxParts, "qgemm_attn: attn_splits %d out of 1..%d",
                attn_splits, cir::kAttnMaxParts);
  CIR_CHECK_ARG(splits >= 1 && (k / 128) % splits == 0, "qgemm_attn: splits (%d) must divide k/128 (%d)", splits,
                k / 128);
  CIR_CHECK_ARG(cir::gemv_fits(m, k, splits), "qgemm_attn: m %d with %d quads per split exceeds the GEMV stage", m,
                (k / 128) / splits);
  CIR_CHECK_ARG(attn_part_o && attn_part_ml && w_tiled && y_partial, "qgemm_attn: null pointer");
  const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
  const uint8_t* q = static_cast<const uint8_t*>(w_tiled);
  const uint16_t* d = reinterpret_cast<const uint16_t*>(q + tiles * 64 * quant_bytes_per_lane(fmt));
  const cir::AttnParts ap{attn_part_o, attn_part_ml, attn_splits, num_heads};
  hipStream_t s = as_stream(stream);
  if (fmt == CIR_Q4_0)
    cir::launch_qgemv<CIR_Q4_0, 0, float, true>(nullptr, k, q, d, y_partial, m, n, k, splits, s, nullptr, ap);
  else
    cir::launch_qgemv<CIR_Q8_0, 0, float, true>(nullptr, k, q, d, y_partial, m, n, k, splits, s, nullptr, ap);
  return launch_status();
}

extern "C" int cir_qgemm_swiglu(const void* x, int ldx, const void* w_tiled, int fmt, void* out, int odt, int m,
                                int inter, int k, void* stream) {
  CIR_CHECK_ARG(valid_fmt(fmt), "qgemm_swiglu: unknown weight format %d", fmt);
  CIR_CHECK_ARG(odt == CIR_F16 || odt == CIR_F32, "qgemm_swiglu: out dtype must be CIR_F16 or CIR_F32");
  CIR_CHECK_ARG(m >= 0 && inter >= 0 && k >= 0, "qgemm_swiglu: negative size");
  if (m == 0 || inter == 0) return 0;
  CIR_CHECK_ARG(inter % 16 == 0, "qgemm_swiglu: intermediate size (%d) must be a multiple of 16", inter);
  CIR_CHECK_ARG(k > 0 && k % 128 == 0, "qgemm_swiglu: k (%d) must be a positive multiple of 128", k);
  CIR_CHECK_ARG(ldx >= k && ldx % 8 == 0, "qgemm_swiglu: ldx (%d) must be >= k and a multiple of 8", ldx);
  CIR_CHECK_ARG(x && w_tiled && out, "qgemm_swiglu: null pointer");
  CIR_CHECK_ARG((m + 15) / 16 <= 65535, "qgemm_swiglu: grid too large");
  const int n = 2 * inter;
  const size_t tiles = (size_t)(n / 16) * (k / 128);
  const uint8_t* q = static_cast<const uint8_t*>(w_tiled);
  const uint16_t* d = reinterpret_cast<const uint16_t*>(q + tiles * 64 * quant_bytes_per_lane(fmt));
  const f16* xh = static_cast<const f16*>(x);
  hipStream_t s = as_stream(stream);
  auto go = [&]<int FMT>() {
    if constexpr (!is_row_fmt(FMT)) {
      if (use_xw_swiglu(m)) {
        auto xw = [&]<int MT>() {
          if (odt == CIR_F16) launch_qgemm_xw_swiglu<FMT, MT, f16>(xh, ldx, q, d, static_cast<f16*>(out), m, n, k, s);
          else launch_qgemm_xw_swiglu<FMT, MT, float>(xh, ldx, q, d, static_cast<float*>(out), m, n, k, s);
        };
        if (m <= 64) xw.template operator()<4>();
        else xw.template operator()<8>();
        return;
      }
    }
    if (use_xl(m, n, k, false)) {
      auto xl = [&]<int MT>() {
        if (odt == CIR_F16) launch_qgemm_xl<FMT, MT, 1, f16>(xh, ldx, q, d, nullptr, m, n, k, 1, s, static_cast<f16*>(out));
        else launch_qgemm_xl<FMT, MT, 1, float>(xh, ldx, q, d, nullptr, m, n, k, 1, s, static_cast<float*>(out));
      };
      if (xl_mt_swiglu(m) == 4) xl.template operator()<4>();
      else xl.template operator()<8>();
      return;
    }
    if (odt == CIR_F16) {
      if (m <= 16) launch_qgemm_swiglu<FMT, 1>(xh, ldx, q, d, static_cast<f16*>(out), m, n, k, s);
      else launch_qgemm_swiglu<FMT, 2>(xh, ldx, q, d, static_cast<f16*>(out), m, n, k, s);
    } else {
      if (m <= 16) launch_qgemm_swiglu<FMT, 1>(xh, ldx, q, d, static_cast<float*>(out), m, n, k, s);
      else launch_qgemm_swiglu<FMT, 2>(xh, ldx, q, d, static_cast<float*>(out), m, n, k, s);
    }
  };
  if (fmt == CIR_Q4_0) go.template operator()<CIR_Q4_0>();
  else if (fmt == CIR_Q8_0) go.template operator()<CIR_Q8_0>();
  else if (fmt == CIR_I4_ROW) go.template operator()<CIR_I4_ROW>();
  else go.template operator()<CIR_I8_ROW>();
  return launch_status();
}

extern "C" int cir_gemm_f32(const float* x, int ldx, const float* w, float* y_partial, int m, int n, int k, int splits,
                            void* stream) {
  CIR_CHECK_ARG(m >= 0 && n >= 0 && k >= 0, "gemm_f32: negative size");
  if (m == 0 || n == 0) return 0;
  CIR_CHECK_ARG(k > 0 && splits >= 1 && splits <= k, "gemm_f32: bad k/splits");
  CIR_CHECK_ARG(ldx >= k, "gemm_f32: ldx (%d) < k (%d)", ldx, k);
  CIR_CHECK_ARG(x && w && y_partial, "gemm_f32: null pointer");
  const int kc = (k + splits - 1) / splits;
  dim3 grid((n + 3) / 4, splits);
  gemm_f32_kernel<<<grid, 256, 0, as_stream(stream)>>>(x, ldx, w, y_partial, m, n, k, kc);
  return launch_status();
}

extern "C" size_t cir_qgemm_argmax_workspace_bytes(int m, int n) {
  if (m <= 0 || n <= 0) return 0;
  return cir::argmax_cand_count(m, n) * (sizeof(float) + sizeof(int));
}

extern "C" int cir_qgemm_argmax(const void* x, int ldx, const void* w_tiled, int fmt, int64_t* ids, void* workspace,
                                size_t ws_bytes, int m, int n, int k, void* stream) {
  CIR_CHECK_ARG(valid_fmt(fmt), "qgemm_argmax: unknown weight format %d", fmt);
  CIR_CHECK_ARG(m >= 0 && n > 0 && k >= 0, "qgemm_argmax: bad sizes (m %d, n %d)", m, n);
  if (m == 0) return 0;
  CIR_CHECK_ARG(k > 0 && k % 128 == 0, "qgemm_argmax: k (%d) must be a positive multiple of 128", k);
  CIR_CHECK_ARG(ldx >= k && ldx % 8 == 0, "qgemm_argmax: ldx (%d) must be >= k and a multiple of 8", ldx);
  CIR_CHECK_ARG(x && w_tiled && ids && workspace, "qgemm_argmax: null pointer");
  CIR_CHECK_ARG(m <= 65535 && (m + 15) / 16 <= 65535, "qgemm_argmax: m (%d) too large", m);
  const size_t cand = cir::argmax_cand_count(m, n);
  CIR_CHECK_ARG(ws_bytes >= cand * (sizeof(float) + sizeof(int)), "qgemm_argmax: workspace needs %zu bytes (got %zu)",
                cand * (sizeof(float) + sizeof(int)), ws_bytes);
  const size_t tiles = (size_t)((n + 15) / 16) * (k / 128);
  const uint8_t* q = static_cast<const uint8_t*>(w_tiled);
  const uint16_t* d = reinterpret_cast<const uint16_t*>(q + tiles * 64 * quant_bytes_per_lane(fmt));
  const f16* xh = static_cast<const f16*>(x);
  float* cv = static_cast<float*>(workspace);
  int* ci = reinterpret_cast<int*>(cv + cand);
  hipStream_t s = as_stream(stream);
  auto go = [&]<int FMT>() {
    if constexpr (!is_row_fmt(FMT)) {
      if (gemv_head_fits(FMT, m, k)) {
        const int tw = launch_qgemv<FMT, 2, int>(xh, ldx, q, d, cv, m, n, k, 1, s, ci);
        argmax_cand_kernel<<<m, 256, 0, s>>>(cv, ci, tw, m, ids);
        return;
      }
    }
    if (use_xl(m, n, k, false)) {
      if (m <= 64) launch_qgemm_xl_argmax<FMT, 4>(xh, ldx, q, d, cv, ci, ids, m, n, k, s);
      else launch_qgemm_xl_argmax<FMT, 8>(xh, ldx, q, d, cv, ci, ids, m, n, k, s);
    } else if (m <= 16) {
      launch_qgemm_argmax<FMT, 1, 1>(xh, ldx, q, d, cv, ci, ids, m, n, k, s);
    } else {
      launch_qgemm_argmax<FMT, 2, 2>(xh, ldx, q, d, cv, ci, ids, m, n, k, s);
    }
  };
  if (fmt == CIR_Q4_0) go.template operator()<CIR_Q4_0>();
  else if (fmt == CIR_Q8_0) go.template operator()<CIR_Q8_0>();
  else if (fmt == CIR_I4_ROW) go.template operator()<CIR_I4_ROW>();
  else go.template operator()<CIR_I8_ROW>();
  return launch_status();
}

extern "C" const char* cir_qgemm_plan(int op, int fmt, int m, int n, int k, int splits) {
  if (!valid_fmt(fmt) || m <= 0 || n <= 0 || k <= 0 || k % 128) return "invalid";
  switch (op) {
    case CIR_GEMM_PARTIALS:
      if (!splits_ok(m, n, k, splits)) return "invalid";
      if (gemv_fits(m, k, splits)) return "qgemv_kernel";
      if (m <= 16) return "qgemm_xs_kernel<NT=1,MT=1>";
      if (!use_xl(m, n, k)) return "qgemm_xs_kernel<NT=2,MT=2>";
      return m <= 64 ? "qgemm_xl_kernel<MT=4>" : "qgemm_xl_kernel<MT=8>";
    case CIR_GEMM_SWIGLU:
      if (!is_row_fmt(fmt) && use_xw_swiglu(m))
        return m <= 64 ? "qgemm_xw_kernel<MT=4,EPI=swiglu>" : "qgemm_xw_kernel<MT=8,EPI=swiglu>";
      if (use_xl(m, n, k, false))
        return xl_mt_swiglu(m) == 4 ? "qgemm_xl_kernel<MT=4,EPI=swiglu>" : "qgemm_xl_kernel<MT=8,EPI=swiglu>";
      return m <= 16 ? "qgemm_xs_kernel<NT=2,MT=1,EPI=swiglu>" : "qgemm_xs_kernel<NT=2,MT=2,EPI=swiglu>";
    case CIR_GEMM_ARGMAX:
      if (gemv_head_fits(fmt, m, k)) return "qgemv_kernel<EPI=argmax>+argmax_cand_kernel";
      if (use_xl(m, n, k, false))
        return m <= 64 ? "qgemm_xl_kernel<MT=4,EPI=argmax>+argmax_cand_kernel"
                       : "qgemm_xl_kernel<MT=8,EPI=argmax>+argmax_cand_kernel";
      return m <= 16 ? "qgemm_xs_kernel<NT=1,MT=1,EPI=argmax>+argmax_cand_kernel"
                     : "qgemm_xs_kernel<NT=2,MT=2,EPI=argmax>+argmax_cand_kernel";
    case CIR_GEMM_ATTN_MERGE:
      if ((fmt != CIR_Q4_0 && fmt != CIR_Q8_0) || splits < 1 || (k / 128) % splits || !gemv_fits(m, k, splits))
        return "invalid";
      return "qgemv_kernel<input=attention partials>";
    default:
      return "invalid";
  }
}
