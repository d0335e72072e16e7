// Fused message GEMM kernels for lmax = 2, bf16, input gradient.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 2, 2, BF16, BWD_DX)
MALOQ_GEMM_BWD_EDGE_INSTANCES(, 2, 2, BF16)

}  // namespace msg
}  // namespace maloq
