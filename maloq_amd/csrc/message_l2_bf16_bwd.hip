// Fused message GEMM kernels for lmax = 2, bf16, input gradient.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 2, 2, BF16, BWD_DX)

}  // namespace msg
}  // namespace maloq
