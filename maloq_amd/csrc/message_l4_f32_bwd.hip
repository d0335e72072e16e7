// Fused message GEMM kernels for lmax = 4, f32, input gradient.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 4, 2, F32, BWD_DX)

}  // namespace msg
}  // namespace maloq
