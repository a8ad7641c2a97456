// Read-bandwidth calibration for the roofline figures: how fast can one kernel on this
// GPU read B bytes from HBM?  bench.py times this launch over buffers rotated past the
// 256 MB MALL, for the byte counts of the hot kernels (a config-3 projection, the
// config-4 gate|up weights, one config-4 attention launch), and reports each hot
// kernel's rate against the best read of the same size beside its fraction of the
// 8 TB/s peak.  Not on the decode path.
#include "common.hpp"

namespace cir {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kReadUnroll = 8;  // 16-byte loads per thread in flight

// layout 0: grid-stride (consecutive threads read consecutive 16-byte chunks across the
// whole buffer); layout 1: each workgroup reads one contiguous chunk.  Every loaded word
// is folded into one value, written only if it equals a constant no input produces, so
// the loads stay.
// side (optional, side16 chunks of 16 B, a power of two): a small buffer that stays in L2, read alongside -- per
// step each thread also loads `side_ratio` chunks of it for every kReadUnroll chunks of the stream, all issued
// before any is consumed: the pattern of a GEMM that streams weights from HBM and re-reads its activations.
__global__ __launch_bounds__(1024) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16, int layout,
                                                           const u32x4* __restrict__ side, uint32_t side16,
                                                           int side_ratio, uint32_t* __restrict__ out) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  size_t i, step, end;
  if (layout == 0) {
    i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    step = (size_t)gridDim.x * blockDim.x;
    end = n16;
  } else {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t begin = per * blockIdx.x;
    i = begin + threadIdx.x;
    step = blockDim.x;
    end = begin + per < n16 ? begin + per : n16;
  }
  uint32_t it = 0;
  for (; i + (kReadUnroll - 1) * step < end; i += kReadUnroll * step, ++it) {
    u32x4 v[kReadUnroll], a[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * step);
    if (side_ratio > 0) {  // uniform branch: the side loads go out before either batch is consumed
#pragma unroll
      for (int u = 0; u < kReadUnroll; ++u)
        if (u < side_ratio) a[u] = side[((it * kReadUnroll + u) * blockDim.x + threadIdx.x) & (side16 - 1)];
#pragma unroll
      for (int u = 0; u < kReadUnroll; ++u)
        if (u < side_ratio) acc ^= a[u];
    }
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u];
  }
  for (; i < end; i += step) acc ^= p[i];
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9E3779B9u && acc.x == 0x7F4A7C15u) out[0] = acc.y;
}

}  // namespace
}  // namespace cir

using namespace cir;

extern "C" int cir_stream_read(const void* buf, size_t bytes, int workgroups, int threads, int layout,
                               const void* side, size_t side_bytes, int side_ratio, void* out, void* stream) {
  CIR_CHECK_ARG(workgroups >= 1 && workgroups <= 65535 && threads >= 64 && threads <= 1024 && threads % 64 == 0 &&
                    (layout == 0 || layout == 1),
                "stream_read: bad launch shape (%d x %d, layout %d)", workgroups, threads, layout);
  const size_t side16 = side_bytes / 16;
  CIR_CHECK_ARG(side_ratio >= 0 && side_ratio <= kReadUnroll, "stream_read: side_ratio %d out of 0..%d", side_ratio,
                kReadUnroll);
  CIR_CHECK_ARG(side_ratio == 0 || (side && side16 > 0 && (side16 & (side16 - 1)) == 0 && side16 <= (1u << 30)),
                "stream_read: the side buffer must hold a power of two of 16-byte chunks");
  if (bytes < 16) return 0;
  CIR_CHECK_ARG(buf && out, "stream_read: null pointer");
  stream_read_kernel<<<workgroups, threads, 0, as_stream(stream)>>>(
      static_cast<const u32x4*>(buf), bytes / 16, layout, static_cast<const u32x4*>(side), (uint32_t)side16,
      side_ratio, static_cast<uint32_t*>(out));
  return launch_status();
}
