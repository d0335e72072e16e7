// Instantiations of the fused message kernel for lmax = 4.
#include "message_launch.h"

namespace maloq {
namespace msg {

int launch_l4(int mmax, int dtype, int gate, int mode, const Args& a, hipStream_t s) {
  MALOQ_REQUIRE(mmax == 2, "lmax=4: built for mmax = 2 only, got %d", mmax);
  return launch_lm<4, 2>(dtype, gate, mode, a, s);
}

int prep_l4(int mmax, int dtype, int mode, const PrepArgs& a, hipStream_t s) {
  MALOQ_REQUIRE(mmax == 2, "lmax=4: built for mmax = 2 only, got %d", mmax);
  return prep_lm<4, 2>(dtype, mode, a, s);
}

}  // namespace msg
}  // namespace maloq
