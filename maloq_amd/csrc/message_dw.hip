// Weight gradients of the SO(2) linear (gfx950).
//
// With Y_e the rotated, radially scaled input rows and dZ_e the rotated output
// gradient rows of edge e (both saved in m-major order [E, d', C] by the
// fused kernels), the gradient of every |m| group is a GEMM with the edges as
// the reduction axis:  C_g = sum_e dZ_g(e)^T Y_g(e), g = 0..mmax.
// Workgroups own 64x64 output tiles of one group and a contiguous edge range
// (split-K); both operands are loaded edge-major (coalesced along channels)
// and transposed through LDS into MFMA fragments.  Partial tiles are summed in
// split order by dw_reduce_kernel, which also folds the +-m quadrants of
// C_m back into the reference layout of so2_m_conv.fc.weight:
//   dWr = C[+,+] + C[-,-],   dWi = C[-,+] - C[+,-]      (so2_layers.py:61-67).
// Deterministic: no atomics.
#include "message_impl.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace msg {

constexpr int MAXG = 8;

struct DwArgs {
  const void* dz;       // [E, dp, C_out]
  const void* y;        // [E, dp, C_in]
  int64_t E;
  int dp, C_out, C_in, ngroups, splits;
  int row0[MAXG], rows[MAXG];
  int ntk[MAXG];             // 64-wide tiles along k (= rows * C_in)
  int64_t tile0[MAXG + 1];   // cumulative tile counts
  int64_t goff[MAXG + 1];    // element offset of group g in one split's partials
  int64_t e_per_split;
  float* part;               // [splits, goff[ngroups]]
};

template <class TM>
__global__ __launch_bounds__(256) void dw_kernel(DwArgs a) {
  constexpr int KCE = TM::KC;  // edges per K step
  __shared__ alignas(16) char sA[2 * FRAG];
  __shared__ alignas(16) char sB[2 * FRAG];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t ntiles = a.tile0[a.ngroups];
  const int64_t split = blockIdx.x / ntiles;
  const int64_t t = blockIdx.x % ntiles;
  int g = 0;
  while (g + 1 < a.ngroups && t >= a.tile0[g + 1]) ++g;
  const int64_t lt = t - a.tile0[g];
  const int tn = static_cast<int>(lt / a.ntk[g]), tk = static_cast<int>(lt % a.ntk[g]);
  const int Ng = a.rows[g] * a.C_out, Kg = a.rows[g] * a.C_in;
  const int n0 = tn * 64, k0 = tk * 64;
  const int64_t eb = split * a.e_per_split;
  const int64_t ee = (eb + a.e_per_split) < a.E ? (eb + a.e_per_split) : a.E;
  const typename TM::raw* dz = reinterpret_cast<const typename TM::raw*>(a.dz);
  const typename TM::raw* y = reinterpret_cast<const typename TM::raw*>(a.y);
  f32x16 acc;
#pragma unroll
  for (int i = 0; i < 16; ++i) acc[i] = 0.f;
  // staging map: 64 columns x KCE edges per operand; each thread moves 64*KCE/256 values
  constexpr int PER = 64 * KCE / 256;
  for (int64_t e0 = eb; e0 < ee; e0 += KCE) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int q = tid * PER + p;        // 0 .. 64*KCE-1
      const int el = q / 64, c = q % 64;  // edge in chunk, column in tile
      const int64_t e = e0 + el;
      // A: dZ^T rows n
      {
        const int n = n0 + c;
        float v = 0.f;
        if (e < ee && n < Ng) {
          const int row = a.row0[g] + n / a.C_out, co = n % a.C_out;
          v = TM::load(dz + (e * a.dp + row) * a.C_out + co);
        }
        *reinterpret_cast<typename TM::raw*>(sA + (c >> 5) * FRAG + frag_off<TM>(c & 31, el)) =
            TM::cvt(v);
      }
      // B: Y columns k
      {
        const int k = k0 + c;
        float v = 0.f;
        if (e < ee && k < Kg) {
          const int row = a.row0[g] + k / a.C_in, ci = k % a.C_in;
          v = TM::load(y + (e * a.dp + row) * a.C_in + ci);
        }
        *reinterpret_cast<typename TM::raw*>(sB + (c >> 5) * FRAG + frag_off<TM>(c & 31, el)) =
            TM::cvt(v);
      }
    }
    __syncthreads();
    mma(acc, sA + (wave >> 1) * FRAG, sB + (wave & 1) * FRAG, lane, TM{});
    __syncthreads();
  }
  float* out = a.part + split * a.goff[a.ngroups] + a.goff[g];
  const int k = k0 + (wave & 1) * 32 + (lane & 31);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int n = n0 + (wave >> 1) * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    if (n < Ng && k < Kg) out[static_cast<int64_t>(n) * Kg + k] = acc[i];
  }
}

// One thread per element of the reference-layout gradients:
// dW0 [(L+1) C_out, (L+1) C_in], then dW_m [2 (L-m+1) C_out, (L-m+1) C_in].
__global__ void dw_reduce_kernel(DwArgs a, int lmax, float* __restrict__ dw0,
                                 float* __restrict__ dw1, float* __restrict__ dw2,
                                 float* __restrict__ dw3) {
  const int g = blockIdx.y;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t Kg = static_cast<int64_t>(a.rows[g]) * a.C_in;
  const int64_t stride = a.goff[a.ngroups];
  auto C = [&](int64_t n, int64_t k) {
    const float* p = a.part + a.goff[g] + n * Kg + k;
    float s = 0.f;
    for (int sp = 0; sp < a.splits; ++sp) s += p[sp * stride];
    return s;
  };
  if (g == 0) {
    const int64_t Ng = static_cast<int64_t>(a.rows[0]) * a.C_out;
    if (idx >= Ng * Kg) return;
    dw0[idx] = C(idx / Kg, idx % Kg);
    return;
  }
  const int m = g;
  const int64_t nr = lmax - m + 1;  // rows per sign
  const int64_t ho = nr * a.C_out, ki_n = nr * a.C_in;
  if (idx >= 2 * ho * ki_n) return;
  const int64_t r = idx / ki_n, ki = idx % ki_n;
  float v;
  if (r < ho) {  // dWr[ko][ki] = C[+ko][+ki] + C[-ko][-ki]
    v = C(r, ki) + C(ho + r, ki_n + ki);
  } else {       // dWi[ko][ki] = C[-ko][+ki] - C[+ko][-ki]
    const int64_t ko = r - ho;
    v = C(ho + ko, ki) - C(ko, ki_n + ki);
  }
  float* dst = m == 1 ? dw1 : (m == 2 ? dw2 : dw3);
  dst[idx] = v;
}

}  // namespace msg
}  // namespace maloq

using namespace maloq;
using namespace maloq::msg;

static int dw_setup(DwArgs& a, int lmax, int mmax, int64_t E, int c_out, int c_in, int splits) {
  MALOQ_REQUIRE(mmax >= 0 && mmax <= 3 && mmax <= lmax, "mmax out of range for the weight gradient");
  MALOQ_REQUIRE(splits >= 1 && splits <= 64, "splits out of range");
  a.E = E;
  a.C_out = c_out;
  a.C_in = c_in;
  a.ngroups = mmax + 1;
  a.splits = splits;
  int row = 0;
  a.tile0[0] = 0;
  a.goff[0] = 0;
  for (int g = 0; g <= mmax; ++g) {
    const int r = (g == 0) ? (lmax + 1) : 2 * (lmax - g + 1);
    a.row0[g] = row;
    a.rows[g] = r;
    row += r;
    const int64_t Ng = static_cast<int64_t>(r) * c_out, Kg = static_cast<int64_t>(r) * c_in;
    a.ntk[g] = static_cast<int>((Kg + 63) / 64);
    a.tile0[g + 1] = a.tile0[g] + ((Ng + 63) / 64) * a.ntk[g];
    a.goff[g + 1] = a.goff[g] + Ng * Kg;
  }
  a.dp = row;
  a.e_per_split = (E + splits - 1) / splits;
  return MALOQ_OK;
}

extern "C" int64_t maloq_message_dw_partials_floats(int lmax, int mmax, int c_out, int c_in,
                                                    int splits) {
  DwArgs a{};
  if (dw_setup(a, lmax, mmax, 0, c_out, c_in, splits)) return -1;
  return a.goff[a.ngroups] * splits;
}

extern "C" int maloq_message_dw(int dtype, int lmax, int mmax, const void* dz, const void* y,
                                int64_t num_edges, int c_out, int c_in, int splits,
                                float* partials, float* dw0, float* dw1, float* dw2, float* dw3,
                                void* stream) {
  MALOQ_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(num_edges >= 0, "num_edges < 0");
  MALOQ_REQUIRE(c_out > 0 && c_in > 0, "bad channels");
  DwArgs a{};
  int rc = dw_setup(a, lmax, mmax, num_edges, c_out, c_in, splits);
  if (rc) return rc;
  MALOQ_REQUIRE(partials && dw0, "null pointer");
  MALOQ_REQUIRE(mmax < 1 || dw1, "dw1 is null");
  MALOQ_REQUIRE(mmax < 2 || dw2, "dw2 is null");
  MALOQ_REQUIRE(mmax < 3 || dw3, "dw3 is null");
  MALOQ_REQUIRE(num_edges == 0 || (dz && y), "null pointer");
  a.dz = dz;
  a.y = y;
  a.part = partials;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t grid = a.tile0[a.ngroups] * splits;
  MALOQ_REQUIRE(grid < (int64_t(1) << 31), "grid too large");
  if (dtype == 1)
    hipLaunchKernelGGL(dw_kernel<BF16>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(dw_kernel<F32>, dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, a);
  rc = check_launch("dw_kernel");
  if (rc) return rc;
  int64_t maxel = 0;
  for (int g = 0; g <= mmax; ++g) {
    const int64_t el = static_cast<int64_t>(a.rows[g]) * c_out * a.rows[g] * c_in;
    maxel = el > maxel ? el : maxel;
  }
  hipLaunchKernelGGL(dw_reduce_kernel, dim3(static_cast<unsigned>((maxel + 255) / 256), mmax + 1),
                     dim3(256), 0, s, a, lmax, dw0, dw1, dw2, dw3);
  return check_launch("dw_reduce_kernel");
}
