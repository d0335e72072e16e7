// Fused message GEMM kernels for lmax = mmax = 6, bf16, input gradient.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 6, 6, BF16, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(, 6, 6, BF16)

}  // namespace msg
}  // namespace maloq
