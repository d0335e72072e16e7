// Fused message GEMM kernels for lmax = 6, bf16, input gradient.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 6, 2, BF16, BWD_DX)

}  // namespace msg
}  // namespace maloq
