#pragma once
// Host-side launch helpers shared by the per-lmax instantiation files.
#include "message_gemm.h"

namespace maloq {
namespace msg {

// Waves per workgroup, 32-edge row tiles per workgroup and resident
// workgroups per CU (the launch bound) for each shape:
//   mmax < lmax, lmax <= 4 without gate: 4 waves x 64 edges, two workgroups
//     per CU (256 registers per lane);
//   gated, lmax <= 4: 32 edges, except the input gradient (BWD_DX): it has no
//     extra accumulators (a gate's rows are an extra input row type);
//   lmax 6 (mmax < lmax): 64 edges in every mode -- a wave owns one degree,
//     and a gated forward's gate rows go to the eighth wave (GPlan::GW), so
//     each weight fragment serves two row tiles;
//   mmax = lmax (every output degree keeps all 2l + 1 row types, d' = d):
//     32-edge tiles;
//   one workgroup per CU: every lmax > 4 kernel (at two 4-wave workgroups per
//     CU the lmax-6 kernels spilled 128-916 bytes per lane), and at mmax =
//     lmax the gated accumulating forwards (the gate rows are extra
//     accumulators).  At lmax > 4 with mmax < lmax that workgroup has 8 waves:
//     a wave owns at most one output degree, fits 256 registers, and shares
//     its SIMD with a second wave (13-14 % faster at lmax 6 than 4 waves with
//     512 registers each); the other one-per-CU shapes keep 4 waves with
//     their accumulators in AGPRs.
template <int L, int M, bool GATE, int MODE = FWD>
struct Cfg {
  static constexpr bool FULL = M == L && L > 2;
  // lmax > 4 with mmax < lmax: 8 waves, so a wave owns at most one degree and
  // two waves share a SIMD (the one-workgroup-per-CU kernel otherwise has a
  // single wave per SIMD to hide its latencies)
  static constexpr int NW = (L > 4 && !FULL) ? 8 : 4;
  static constexpr int RT = FULL ? 1 : ((MODE == BWD_DX || L > 4 || !GATE) ? 2 : 1);
  static constexpr int MINB = (L > 4 || (FULL && GATE && (MODE == FWD || MODE == FWD_EDGE))) ? 1 : 2;
};

inline int tile_edges(int lmax, int mmax, int gate, int mode = FWD) {
  if (mmax == lmax && lmax > 2) return 32;
  return (mode == BWD_DX || lmax > 4 || !gate) ? 64 : 32;
}
// Every instantiation's tile has a multiple of 32 edges: partial-segment
// buffers sized for 32-edge tiles fit them all.
constexpr int MIN_TILE_EDGES = 32;

template <int L, int M, bool GATE, class TM, int MODE, int KR>
void launch_kr(const Args& a, dim3 g, dim3 b, hipStream_t s) {
  using C = Cfg<L, M, GATE, MODE>;
  if (MODE == BWD_DX && a.rad != nullptr)
    hipLaunchKernelGGL((gemm_kernel<L, M, GATE, C::NW, C::RT, TM, MODE, KR, MODE == BWD_DX, C::MINB>), g, b, 0, s,
                       a);
  else
    hipLaunchKernelGGL((gemm_kernel<L, M, GATE, C::NW, C::RT, TM, MODE, KR, false, C::MINB>), g, b, 0, s, a);
}

template <int L, int M, bool GATE, class TM, class TX, int MODE>
int launch(const Args& a, hipStream_t s) {
  constexpr int NW = Cfg<L, M, GATE, MODE>::NW, RT = Cfg<L, M, GATE, MODE>::RT;
  MALOQ_REQUIRE(tile_edges(L, M, GATE, MODE) == 32 * RT, "tile size mismatch");
  using P = GPlan<L, M, GATE, NW, RT>;
  // Must match the workgroup -> (tile, channel block) mapping of Gemm::run:
  // tiles in groups of 8 (one per XCD), n_cb workgroups per tile.
  const int64_t grid = ((a.ntiles + 7) / 8) * 8 * a.n_cb;
  MALOQ_REQUIRE(grid < (int64_t(1) << 31), "grid too large");
  const dim3 g(static_cast<unsigned>(grid)), b(P::NT);
  // the A-stage ring position of each K step is static per nks % 3 (nks >= 2)
  const int nks = a.C_k / TM::KC;
  switch (nks >= 2 ? nks % 3 : 3) {
    case 0: launch_kr<L, M, GATE, TM, MODE, 0>(a, g, b, s); break;
    case 1: launch_kr<L, M, GATE, TM, MODE, 1>(a, g, b, s); break;
    case 2: launch_kr<L, M, GATE, TM, MODE, 2>(a, g, b, s); break;
    default: launch_kr<L, M, GATE, TM, MODE, 3>(a, g, b, s); break;
  }
  return check_launch("gemm_kernel");
}

// The GEMM instantiations of one (lmax, mmax, dtype, mode), gated and not:
// defined (KW empty) in their own translation unit each, so the per-lmax
// kernel sets compile in parallel, and declared (KW extern) where launch_lm
// dispatches to them.
#define MALOQ_GEMM_INSTANCES(KW, L, M, TM, MODE)                              \
  KW template int launch<L, M, false, TM, TM, MODE>(const Args&, hipStream_t); \
  KW template int launch<L, M, true, TM, TM, MODE>(const Args&, hipStream_t);
// The gated edge-frame forward (first convolution of a two-convolution block).
#define MALOQ_GEMM_EDGE_INSTANCES(KW, L, M, TM) \
  KW template int launch<L, M, true, TM, TM, FWD_EDGE>(const Args&, hipStream_t);
// Its transposed counterpart for the input gradient of the second convolution (ungated).
#define MALOQ_GEMM_BWD_EDGE_INSTANCES(KW, L, M, TM) \
  KW template int launch<L, M, false, TM, TM, BWD_EDGE>(const Args&, hipStream_t);

// dtype: 0 fp32, 1 bf16; mode: FWD, BWD_DX or FWD_EDGE (gated only).
template <int L, int M>
int launch_lm(int dtype, int gate, int mode, const Args& a, hipStream_t s) {
  if (mode == FWD_EDGE) {
    MALOQ_REQUIRE(gate, "the edge-frame forward is built gated only");
    return dtype == 1 ? launch<L, M, true, BF16, BF16, FWD_EDGE>(a, s) : launch<L, M, true, F32, F32, FWD_EDGE>(a, s);
  }
  if (mode == BWD_EDGE) {
    MALOQ_REQUIRE(!gate && a.rad == nullptr && a.gsave != nullptr,
                  "the edge-frame input gradient is built ungated, without radial, with the gate backward");
    return dtype == 1 ? launch<L, M, false, BF16, BF16, BWD_EDGE>(a, s)
                      : launch<L, M, false, F32, F32, BWD_EDGE>(a, s);
  }
  if (mode == FWD) {
    if (dtype == 1)
      return gate ? launch<L, M, true, BF16, BF16, FWD>(a, s) : launch<L, M, false, BF16, BF16, FWD>(a, s);
    return gate ? launch<L, M, true, F32, F32, FWD>(a, s) : launch<L, M, false, F32, F32, FWD>(a, s);
  }
  if (dtype == 1)
    return gate ? launch<L, M, true, BF16, BF16, BWD_DX>(a, s) : launch<L, M, false, BF16, BF16, BWD_DX>(a, s);
  return gate ? launch<L, M, true, F32, F32, BWD_DX>(a, s) : launch<L, M, false, F32, F32, BWD_DX>(a, s);
}

// Edge prep: mode FWD gathers x (dtype) and applies rad; mode BWD_DX gathers
// fp32 output gradients and writes dtype rows.
template <int L, int M>
int prep_lm(int dtype, int mode, const PrepArgs& a, hipStream_t s) {
  const int64_t grid = (a.E + PREP_TE - 1) / PREP_TE;
  MALOQ_REQUIRE(grid < (int64_t(1) << 31), "grid too large");
  const dim3 g(static_cast<unsigned>(grid)), b(PREP_NT);
  const bool gated = mode != FWD && a.gsave != nullptr;
  if (dtype == 1) {
    if (mode == FWD)
      hipLaunchKernelGGL((prep_kernel<L, M, BF16, BF16>), g, b, 0, s, a);
    else if (gated)
      hipLaunchKernelGGL((prep_kernel<L, M, BF16, F32, true>), g, b, 0, s, a);
    else
      hipLaunchKernelGGL((prep_kernel<L, M, BF16, F32>), g, b, 0, s, a);
  } else {
    if (gated)
      hipLaunchKernelGGL((prep_kernel<L, M, F32, F32, true>), g, b, 0, s, a);
    else
      hipLaunchKernelGGL((prep_kernel<L, M, F32, F32>), g, b, 0, s, a);
  }
  return check_launch("prep_kernel");
}

int launch_l2(int mmax, int dtype, int gate, int mode, const Args& a, hipStream_t s);
int launch_l4(int mmax, int dtype, int gate, int mode, const Args& a, hipStream_t s);
int launch_l6(int mmax, int dtype, int gate, int mode, const Args& a, hipStream_t s);
int prep_l2(int mmax, int dtype, int mode, const PrepArgs& a, hipStream_t s);
int prep_l4(int mmax, int dtype, int mode, const PrepArgs& a, hipStream_t s);
int prep_l6(int mmax, int dtype, int mode, const PrepArgs& a, hipStream_t s);

}  // namespace msg
}  // namespace maloq
