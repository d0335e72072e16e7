// Weight gradients of the SO(2) linear (gfx950).
//
// With Y_e the rotated, radially scaled input rows and dZ_e the rotated output
// gradient rows of edge e (both saved in m-major order [E, d', C] by the
// fused kernels), the gradient of every |m| group is a GEMM with the edges as
// the reduction axis:  C_g = sum_e dZ_g(e)^T Y_g(e), g = 0..mmax.
//
// Tiling.  A workgroup (4 waves) owns a 128 x 128 tile of one C_g and a
// contiguous edge range (split-K).  Each K step covers KE edges (64 bf16 /
// 16 fp32): every thread loads one VEC x VEC block (VEC edges x VEC columns,
// one 16-byte load per edge, coalesced along the columns), transposes it in
// registers and writes VEC 16-byte rows straight into MFMA fragment order, so
// both operands are K(edge)-contiguous per lane.  Loads for step s+1 are
// issued before the MFMAs of step s and land in the other LDS buffer (one
// barrier per step).  Each wave computes a 64 x 64 sub-tile (2 x 2 MFMA
// tiles of 32 x 32).  Partial tiles are summed in split order by
// dw_reduce_kernel, which also folds the +-m quadrants of C_m back into the
// reference layout of so2_m_conv.fc.weight:
//   dWr = C[+,+] + C[-,-],   dWi = C[-,+] - C[+,-]      (so2_layers.py:61-67).
// Deterministic: no atomics.
#include "message_impl.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace msg {

constexpr int MAXG = 8;
constexpr int DW_T = 128;  // output tile edge

struct DwArgs {
  const void* dz;       // [E, dp, C_out]
  const void* y;        // [E, dp, C_in]
  int64_t E;
  int dp, C_out, C_in, ngroups, splits;
  int row0[MAXG], rows[MAXG];
  int ntk[MAXG];             // DW_T-wide tiles along k (= rows * C_in)
  int64_t tile0[MAXG + 1];   // cumulative tile counts
  int64_t goff[MAXG + 1];    // element offset of group g in one split's partials
  int64_t e_per_split;       // multiple of the K step
  float* part;               // [splits, goff[ngroups]]
};

template <class TM>
struct DwCfg {
  static constexpr int VEC = TM::VEC;            // elements per 16-byte row
  static constexpr int KC = TM::KC;              // edges per MFMA fragment
  static constexpr int KE = VEC * VEC * 256 / (2 * DW_T);  // edges per K step (1 block per thread)
  static constexpr int NSUB = KE / KC;           // fragment columns per step
  static constexpr int FRAGS = (DW_T / 32) * NSUB;  // fragments per operand per step
  static constexpr int STAGE = 2 * FRAGS * FRAG;    // A + B bytes per step
};

// Transposes a VEC x VEC block held as VEC rows of 16 bytes (row = edge,
// VEC column elements) into VEC rows of VEC edges (row = column).
__device__ __forceinline__ void transpose_block(const uint4 (&in)[8], uint4 (&out)[8], BF16) {
  // 16-bit elements: word w of out[c] = (in[2w] elem c) | (in[2w+1] elem c) << 16
  const uint32_t* iw = reinterpret_cast<const uint32_t*>(in);
  uint32_t* ow = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const uint32_t lo = iw[(2 * w) * 4 + (c >> 1)], hi = iw[(2 * w + 1) * 4 + (c >> 1)];
      // v_perm_b32 selector: bytes of hi are 4..7, bytes of lo 0..3
      const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
      ow[c * 4 + w] = __builtin_amdgcn_perm(hi, lo, sel);
    }
  }
}
__device__ __forceinline__ void transpose_block(const uint4 (&in)[4], uint4 (&out)[4], F32) {
  const uint32_t* iw = reinterpret_cast<const uint32_t*>(in);
  uint32_t* ow = reinterpret_cast<uint32_t*>(out);
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 4; ++e) ow[c * 4 + e] = iw[e * 4 + c];
}

template <class TM>
__global__ __launch_bounds__(256) void dw_kernel(DwArgs a) {
  using Cfg = DwCfg<TM>;
  constexpr int VEC = Cfg::VEC, KE = Cfg::KE, NSUB = Cfg::NSUB;
  __shared__ alignas(16) char smem[2 * Cfg::STAGE];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t ntiles = a.tile0[a.ngroups];
  const int64_t split = blockIdx.x / ntiles;
  const int64_t t = blockIdx.x % ntiles;
  int g = 0;
  while (g + 1 < a.ngroups && t >= a.tile0[g + 1]) ++g;
  const int64_t lt = t - a.tile0[g];
  const int tn = static_cast<int>(lt / a.ntk[g]), tk = static_cast<int>(lt % a.ntk[g]);
  const int Ng = a.rows[g] * a.C_out, Kg = a.rows[g] * a.C_in;
  const int64_t eb = split * a.e_per_split;
  const int64_t ee = (eb + a.e_per_split) < a.E ? (eb + a.e_per_split) : a.E;

  // this thread's block: operand (0 = dZ -> A, 1 = Y -> B), column group, edge group
  const int op = tid >> 7;
  const int bi = tid & 127;
  const int cg = bi % (DW_T / VEC), eg = bi / (DW_T / VEC);
  const int C = op ? a.C_in : a.C_out;
  const int col = (op ? tk : tn) * DW_T + cg * VEC;   // first column of the block in C_g
  const int lim = op ? Kg : Ng;
  const typename TM::raw* src = reinterpret_cast<const typename TM::raw*>(op ? a.y : a.dz);
  int64_t coladdr = -1;  // element offset of (edge 0, col) or -1 if the block is outside the tile
  if (col < lim) coladdr = static_cast<int64_t>(a.row0[g] + col / C) * C + col % C;
  const int64_t estride = static_cast<int64_t>(a.dp) * C;
  // LDS destination: fragment (col tile, k-substep), row = column within the tile
  const int cl = cg * VEC;  // column within the 128 tile
  const int e_in = eg * VEC;
  const int frag = op * Cfg::FRAGS + (cl >> 5) * NSUB + e_in / TM::KC;
  const int lds_off = frag * FRAG + frag_off<TM>(cl & 31, e_in % TM::KC);  // + c * row pitch below

  uint4 regs[VEC];
  auto load = [&](int64_t e0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      const int64_t e = e0 + e_in + v;
      regs[v] = make_uint4(0u, 0u, 0u, 0u);
      if (coladdr >= 0 && e < ee) regs[v] = *reinterpret_cast<const uint4*>(src + e * estride + coladdr);
    }
  };
  auto store = [&](int buf) {
    uint4 tr[VEC];
    transpose_block(regs, tr, TM{});
    char* base = smem + buf * Cfg::STAGE + lds_off;
#pragma unroll
    for (int c = 0; c < VEC; ++c)
      *reinterpret_cast<uint4*>(base + frag_off<TM>(c, 0) - frag_off<TM>(0, 0)) = tr[c];
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int wn = wave >> 1, wk = wave & 1;
  const int64_t nsteps = ee > eb ? (ee - eb + KE - 1) / KE : 0;
  if (nsteps > 0) {
    load(eb);
    store(0);
  }
  __syncthreads();
  for (int64_t s = 0; s < nsteps; ++s) {
    const bool more = s + 1 < nsteps;
    if (more) load(eb + (s + 1) * KE);
    const char* A = smem + (s & 1) * Cfg::STAGE;
    const char* B = A + Cfg::FRAGS * FRAG;
#pragma unroll
    for (int ks = 0; ks < NSUB; ++ks) {
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          mma(acc[i][j], A + ((2 * wn + i) * NSUB + ks) * FRAG, B + ((2 * wk + j) * NSUB + ks) * FRAG,
              lane, TM{});
    }
    if (more) store((s + 1) & 1);
    __syncthreads();
  }
  float* out = a.part + split * a.goff[a.ngroups] + a.goff[g];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int k = tk * DW_T + (2 * wk + j) * 32 + (lane & 31);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int n = tn * DW_T + (2 * wn + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
        if (n < Ng && k < Kg) out[static_cast<int64_t>(n) * Kg + k] = acc[i][j][r];
      }
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
    a.ntk[g] = static_cast<int>((Kg + DW_T - 1) / DW_T);
    a.tile0[g + 1] = a.tile0[g] + ((Ng + DW_T - 1) / DW_T) * a.ntk[g];
    a.goff[g + 1] = a.goff[g] + Ng * Kg;
  }
  a.dp = row;
  // split boundaries on a multiple of the largest K step (64 edges)
  a.e_per_split = ((E + splits - 1) / splits + 63) / 64 * 64;
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
