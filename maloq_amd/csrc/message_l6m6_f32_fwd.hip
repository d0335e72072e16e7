// Fused message GEMM kernels for lmax = mmax = 6, f32, forward.
#include "message_launch.h"

namespace maloq {
namespace msg {

MALOQ_GEMM_INSTANCES(, 6, 6, F32, FWD)
MALOQ_GEMM_EDGE_INSTANCES(, 6, 6, F32)

}  // namespace msg
}  // namespace maloq
