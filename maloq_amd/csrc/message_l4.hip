// Prep kernels and the GEMM dispatch of the fused message block for lmax = 4
// (mmax = 2, the benchmark's truncation, and mmax = 4, the reference models').
#include "message_launch.h"

namespace maloq {
namespace msg {

// GEMM kernels: defined in message_l4_<dtype>_<mode>.hip (mmax 2) and
// message_l4m4_<dtype>_<mode>.hip (mmax 4)
MALOQ_GEMM_INSTANCES(extern, 4, 2, BF16, FWD)
MALOQ_GEMM_EDGE_INSTANCES(extern, 4, 2, BF16)
MALOQ_GEMM_INSTANCES(extern, 4, 2, BF16, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(extern, 4, 2, BF16)
MALOQ_GEMM_INSTANCES(extern, 4, 2, F32, FWD)
MALOQ_GEMM_EDGE_INSTANCES(extern, 4, 2, F32)
MALOQ_GEMM_INSTANCES(extern, 4, 2, F32, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(extern, 4, 2, F32)
MALOQ_GEMM_INSTANCES(extern, 4, 4, BF16, FWD)
MALOQ_GEMM_EDGE_INSTANCES(extern, 4, 4, BF16)
MALOQ_GEMM_INSTANCES(extern, 4, 4, BF16, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(extern, 4, 4, BF16)
MALOQ_GEMM_INSTANCES(extern, 4, 4, F32, FWD)
MALOQ_GEMM_EDGE_INSTANCES(extern, 4, 4, F32)
MALOQ_GEMM_INSTANCES(extern, 4, 4, F32, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(extern, 4, 4, F32)

int launch_l4(int mmax, int dtype, int gate, int mode, const Args& a, hipStream_t s) {
  if (mmax == 2) return launch_lm<4, 2>(dtype, gate, mode, a, s);
  if (mmax == 4) return launch_lm<4, 4>(dtype, gate, mode, a, s);
  MALOQ_REQUIRE(false, "lmax=4: built for mmax 2 and 4, got %d", mmax);
}

int prep_l4(int mmax, int dtype, int mode, const PrepArgs& a, hipStream_t s) {
  if (mmax == 2) return prep_lm<4, 2>(dtype, mode, a, s);
  if (mmax == 4) return prep_lm<4, 4>(dtype, mode, a, s);
  MALOQ_REQUIRE(false, "lmax=4: built for mmax 2 and 4, got %d", mmax);
}

}  // namespace msg
}  // namespace maloq
