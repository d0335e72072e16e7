// Prep kernels and the GEMM dispatch of the fused message block for lmax = 2.
#include "message_launch.h"

namespace maloq {
namespace msg {

// GEMM kernels: defined in message_l2_<dtype>_<mode>.hip
MALOQ_GEMM_INSTANCES(extern, 2, 2, BF16, FWD)
MALOQ_GEMM_EDGE_INSTANCES(extern, 2, 2, BF16)
MALOQ_GEMM_INSTANCES(extern, 2, 2, BF16, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(extern, 2, 2, BF16)
MALOQ_GEMM_INSTANCES(extern, 2, 2, F32, FWD)
MALOQ_GEMM_EDGE_INSTANCES(extern, 2, 2, F32)
MALOQ_GEMM_INSTANCES(extern, 2, 2, F32, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(extern, 2, 2, F32)

int launch_l2(int mmax, int dtype, int gate, int mode, const Args& a, hipStream_t s) {
  MALOQ_REQUIRE(mmax == 2, "lmax=2: built for mmax = 2 only, got %d", mmax);
  return launch_lm<2, 2>(dtype, gate, mode, a, s);
}

int prep_l2(int mmax, int dtype, int mode, const PrepArgs& a, hipStream_t s) {
  MALOQ_REQUIRE(mmax == 2, "lmax=2: built for mmax = 2 only, got %d", mmax);
  return prep_lm<2, 2>(dtype, mode, a, s);
}

}  // namespace msg
}  // namespace maloq
