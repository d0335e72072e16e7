// Fused message GEMM kernels for lmax = mmax = 4, f32, forward.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 4, 4, F32, FWD)
MALOQ_GEMM_EDGE_INSTANCES(, 4, 4, F32)

}  // namespace msg
}  // namespace maloq
