// Deterministic sorted-segment sum (gfx950).
//
// Replaces the float-atomic index_add_ of the reference
// (helm/esen_block.py:194-206, helm/nn/embedding.py:129-131): edges are
// grouped by destination (CSR seg_ptr over a permutation), and each output
// element is summed in edge order by one thread, so results are bitwise
// reproducible run to run.  HBM-bound: one read of every message element, one
// write of every node element; float4 accesses along the feature axis.
#include "common.h"
#include "../../include/maloq_hip.h"

namespace maloq {

__global__ __launch_bounds__(256) void segment_sum_kernel(const float* __restrict__ msg,
                                                          const int64_t* __restrict__ perm,
                                                          const int64_t* __restrict__ seg_ptr,
                                                          int64_t width, float* __restrict__ out) {
  const int64_t n = blockIdx.y;
  const int64_t c4 = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (c4 >= width) return;
  const int64_t p0 = seg_ptr[n], p1 = seg_ptr[n + 1];
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (c4 + 4 <= width && (width % 4) == 0) {
    for (int64_t p = p0; p < p1; ++p) {
      const int64_t e = perm ? perm[p] : p;
      const float4 v = *reinterpret_cast<const float4*>(msg + e * width + c4);
      acc.x += v.x; acc.y += v.y; acc.z += v.z; acc.w += v.w;
    }
    *reinterpret_cast<float4*>(out + n * width + c4) = acc;
  } else {
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    for (int64_t p = p0; p < p1; ++p) {
      const int64_t e = perm ? perm[p] : p;
      for (int q = 0; q < 4; ++q)
        if (c4 + q < width) a[q] += msg[e * width + c4 + q];
    }
    for (int q = 0; q < 4; ++q)
      if (c4 + q < width) out[n * width + c4 + q] = a[q];
  }
}

}  // namespace maloq

extern "C" int maloq_segment_sum(const float* msg, const int64_t* perm, const int64_t* seg_ptr,
                                 int64_t num_segments, int64_t width, float* out, void* stream) {
  MALOQ_REQUIRE(num_segments >= 0 && width >= 0, "bad sizes");
  if (num_segments == 0 || width == 0) return MALOQ_OK;
  MALOQ_REQUIRE(seg_ptr && out, "null pointer");
  MALOQ_REQUIRE(num_segments < 65536 * 32768LL, "too many segments");
  const int64_t cols4 = (width + 3) / 4;
  const unsigned gx = static_cast<unsigned>((cols4 + 255) / 256);
  // gridDim.y is limited to 65535: fold extra segments into repeated launches.
  const int64_t chunk = 65535;
  for (int64_t s0 = 0; s0 < num_segments; s0 += chunk) {
    const int64_t ns = (num_segments - s0) < chunk ? (num_segments - s0) : chunk;
    hipLaunchKernelGGL(maloq::segment_sum_kernel, dim3(gx, static_cast<unsigned>(ns)), dim3(256),
                       0, static_cast<hipStream_t>(stream), msg, perm, seg_ptr + s0, width,
                       out + s0 * width);
    int rc = maloq::check_launch("segment_sum_kernel");
    if (rc) return rc;
  }
  return MALOQ_OK;
}
