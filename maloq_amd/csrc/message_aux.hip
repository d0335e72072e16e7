// Small device helpers of the fused message block's host side (gfx950):
//   * weight packing: the SO(2) weights (fc_m0 and the so2_m_conv fc matrices,
//     fp32, reference layout) gathered into the MFMA-fragment order of the
//     GEMM kernels and converted to the operand type in one launch;
//   * bias gradient: column sums over edges of chosen rows of the saved
//     output-gradient rows (dL/db0 of fc_m0), split over edge ranges and
//     summed in a fixed order (deterministic, no atomics);
//   * kept Wigner rows from a caller's dense [E, d, d] wigner, in the pair
//     layout the fused kernels read (PairLayout in message_impl.h).
#include "message_impl.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace aux {

constexpr int MAXSRC = 8;  // fc_m0 and so2_m_conv[m - 1] for m <= 7

struct PackArgs {
  const float* src[MAXSRC];
  int64_t end[MAXSRC];  // cumulative element counts of the sources
  int nsrc;
  const int64_t* idx;   // [n] flat index into the concatenated sources
  int64_t n;
  void* out;
};

template <bool BF>
__global__ void pack_kernel(PackArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= a.n) return;
  const int64_t j = a.idx[i];
  int k = 0;
  while (k + 1 < a.nsrc && j >= a.end[k]) ++k;
  const float v = a.src[k][j - (k > 0 ? a.end[k - 1] : 0)];
  if constexpr (BF)
    reinterpret_cast<uint16_t*>(a.out)[i] = f32_to_bf16(v);
  else
    reinterpret_cast<float*>(a.out)[i] = v;
}

// Column sums of a row set, one level of a fixed-order tree: block (x, s)
// sums rows [s RB, (s + 1) RB) of columns [64 VEC x, 64 VEC (x + 1)) and writes
// dst[s][col].  Row r of the source starts at src + off + r * stride
// elements; the n columns are contiguous.  Thread (tx, ty) adds rows
// ty, ty + 4, ... of the block's range in order, then the four ty partials are
// added in order through LDS: the result depends only on the row count.
constexpr int CS_RB = 64;   // rows per block
constexpr int CS_TY = 4;    // row lanes per block
constexpr int CS_TX = 64;   // column vectors per block

template <bool BF>
__global__ __launch_bounds__(CS_TX * CS_TY) void colsum_kernel(const void* __restrict__ src, int64_t off,
                                                               int64_t stride, int64_t n, int64_t rows,
                                                               float* __restrict__ dst) {
  constexpr int VEC = BF ? 8 : 4;  // 16 bytes per load
  constexpr int PER = CS_RB / CS_TY;
  __shared__ float red[CS_TY - 1][CS_TX][VEC + 1];
  const int tx = threadIdx.x % CS_TX, ty = threadIdx.x / CS_TX;
  const int64_t col = (static_cast<int64_t>(blockIdx.x) * CS_TX + tx) * VEC;
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * CS_RB;
  const bool live = col < n;
  const int64_t colc = live ? col : 0;
  float acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; ++v) acc[v] = 0.f;
  if (rows > 0) {
    uint4 buf[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      int64_t r = r0 + ty + CS_TY * i;
      r = r < rows ? r : rows - 1;  // clamped: every load is in bounds
      const char* p = static_cast<const char*>(src) + (off + r * stride + colc) * (BF ? 2 : 4);
      buf[i] = *reinterpret_cast<const uint4*>(p);
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      if (r0 + ty + CS_TY * i >= rows) continue;
      if constexpr (BF) {
        const uint32_t w[4] = {buf[i].x, buf[i].y, buf[i].z, buf[i].w};
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          acc[2 * v] += __uint_as_float(w[v] << 16);
          acc[2 * v + 1] += __uint_as_float(w[v] & 0xffff0000u);
        }
      } else {
        acc[0] += __uint_as_float(buf[i].x);
        acc[1] += __uint_as_float(buf[i].y);
        acc[2] += __uint_as_float(buf[i].z);
        acc[3] += __uint_as_float(buf[i].w);
      }
    }
  }
  if (ty > 0) {
#pragma unroll
    for (int v = 0; v < VEC; ++v) red[ty - 1][tx][v] = acc[v];
  }
  __syncthreads();
  if (ty == 0 && live) {
    float* d = dst + static_cast<int64_t>(blockIdx.y) * n + col;
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
      float t = acc[v];
#pragma unroll
      for (int j = 0; j < CS_TY - 1; ++j) t += red[j][tx][v];
      d[v] = t;
    }
  }
}

static int64_t cs_blocks(int64_t rows) { return rows <= CS_RB ? 1 : (rows + CS_RB - 1) / CS_RB; }

// dk[p][k] for k in the pair layout of (L, M): D(q, j) of degree l is
// wigner[e][l^2 + i(q)][l^2 + j] with i(0) = l, i(2m - 1) = l + m, i(2m) = l - m
// (the m-major row types), e = perm[p] (or p); padding entries are zero.
template <int L, int M>
__global__ void wigner_rows_kernel(const float* __restrict__ wigner, const int64_t* __restrict__ perm,
                                   int64_t E, float* __restrict__ dk) {
  using PL = msg::PairLayout<L, M>;
  constexpr int WS = PL::WS, d = (L + 1) * (L + 1);
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= E * WS) return;
  const int64_t p = idx / WS;
  const int k = static_cast<int>(idx - p * WS);
  int l = 0;
  while (l < L && k >= PL::woff(l + 1)) ++l;
  const int r = k - PL::woff(l), pb = PL::pblk(l);
  const int pair = r / pb, s = r - pair * pb;
  const int q = s >> 1, j = 2 * pair + (s & 1);
  float v = 0.f;
  if (q < PL::nq(l) && j <= 2 * l) {
    const int m = (q + 1) >> 1;
    const int i = q == 0 ? l : ((q & 1) ? l + m : l - m);
    const int64_t e = perm != nullptr ? perm[p] : p;
    v = wigner[(e * d + l * l + i) * d + l * l + j];
  }
  dk[idx] = v;
}

template <int L, int M>
int wigner_rows(const float* wigner, const int64_t* perm, int64_t E, float* dk, hipStream_t s) {
  const int64_t n = E * msg::PairLayout<L, M>::WS;
  const int64_t grid = (n + 255) / 256;
  MALOQ_REQUIRE(grid < (int64_t(1) << 31), "grid too large");
  hipLaunchKernelGGL((wigner_rows_kernel<L, M>), dim3(static_cast<unsigned>(grid)), dim3(256), 0, s, wigner, perm,
                     E, dk);
  return check_launch("wigner_rows_kernel");
}

}  // namespace aux
}  // namespace maloq

using namespace maloq;
using namespace maloq::aux;

extern "C" int maloq_message_pack(int dtype, int nsrc, const float* const* srcs,
                                  const int64_t* src_sizes, const int64_t* idx, int64_t n, void* out,
                                  void* stream) {
  MALOQ_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(nsrc >= 1 && nsrc <= MAXSRC, "1..%d weight sources", MAXSRC);
  MALOQ_REQUIRE(srcs && src_sizes && n >= 0, "null pointer");
  if (n == 0) return MALOQ_OK;
  MALOQ_REQUIRE(idx && out, "null pointer");
  PackArgs a{};
  int64_t tot = 0;
  for (int k = 0; k < nsrc; ++k) {
    MALOQ_REQUIRE(srcs[k] && src_sizes[k] >= 0, "bad weight source %d", k);
    a.src[k] = srcs[k];
    tot += src_sizes[k];
    a.end[k] = tot;
  }
  a.nsrc = nsrc;
  a.idx = idx;
  a.n = n;
  a.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>((n + 255) / 256);
  if (dtype == 1)
    hipLaunchKernelGGL(pack_kernel<true>, dim3(grid), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(pack_kernel<false>, dim3(grid), dim3(256), 0, s, a);
  return check_launch("pack_kernel");
}

extern "C" int64_t maloq_message_colsum_partials_floats(int nrows, int c, int64_t num_edges) {
  if (nrows <= 0 || c <= 0 || num_edges < 0) return 0;
  const int64_t s1 = cs_blocks(num_edges), s2 = cs_blocks(s1);
  return (s1 > 1 ? s1 : 0) * nrows * c + (s2 > 1 ? s2 : 0) * nrows * c;
}

extern "C" int maloq_message_colsum(int dtype, const void* rows, int rows_per_edge, int row0,
                                    int nrows, int c, int64_t num_edges, float* partials,
                                    float* out, void* stream) {
  MALOQ_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(nrows >= 0 && c > 0 && row0 >= 0 && row0 + nrows <= rows_per_edge, "bad row range");
  MALOQ_REQUIRE(num_edges >= 0, "num_edges < 0");
  const int vec = dtype == 1 ? 8 : 4;
  MALOQ_REQUIRE(c % vec == 0, "channel count %d must be a multiple of %d", c, vec);
  const int64_t n = static_cast<int64_t>(nrows) * c;
  if (n == 0) return MALOQ_OK;
  MALOQ_REQUIRE(out && (num_edges == 0 || rows), "null pointer");
  MALOQ_REQUIRE(partials || maloq_message_colsum_partials_floats(nrows, c, num_edges) == 0,
                "partials workspace required");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // level 0 reads the edge rows; later levels read fp32 partials, ping-ponging
  // between the two halves of the workspace, until one block row remains
  const void* src = rows;
  int64_t off = static_cast<int64_t>(row0) * c, stride = static_cast<int64_t>(rows_per_edge) * c;
  int64_t nr = num_edges;
  bool bf = dtype == 1;
  const int64_t s1 = cs_blocks(num_edges);
  float* half[2] = {partials, partials ? partials + (s1 > 1 ? s1 : 0) * n : nullptr};
  for (int level = 0;; ++level) {
    const int64_t sb = cs_blocks(nr);
    float* dst = sb == 1 ? out : half[level & 1];
    const int64_t vecs = (n + (bf ? 8 : 4) - 1) / (bf ? 8 : 4);
    const dim3 grid(static_cast<unsigned>((vecs + CS_TX - 1) / CS_TX), static_cast<unsigned>(sb));
    if (bf)
      hipLaunchKernelGGL(colsum_kernel<true>, grid, dim3(CS_TX * CS_TY), 0, s, src, off, stride, n, nr, dst);
    else
      hipLaunchKernelGGL(colsum_kernel<false>, grid, dim3(CS_TX * CS_TY), 0, s, src, off, stride, n, nr, dst);
    int rc = check_launch("colsum_kernel");
    if (rc || sb == 1) return rc;
    src = dst;
    off = 0;
    stride = n;
    nr = sb;
    bf = false;
  }
}

extern "C" int maloq_message_wigner_rows(int lmax, int mmax, const float* wigner, const int64_t* perm,
                                         int64_t num_edges, float* dk, void* stream) {
  MALOQ_REQUIRE(maloq_message_supported(lmax, mmax), "no message kernels for lmax %d, mmax %d", lmax, mmax);
  MALOQ_REQUIRE(num_edges >= 0, "num_edges < 0");
  if (num_edges == 0) return MALOQ_OK;
  MALOQ_REQUIRE(wigner && dk, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (lmax * 10 + mmax) {
    case 22: return aux::wigner_rows<2, 2>(wigner, perm, num_edges, dk, s);
    case 42: return aux::wigner_rows<4, 2>(wigner, perm, num_edges, dk, s);
    case 44: return aux::wigner_rows<4, 4>(wigner, perm, num_edges, dk, s);
    case 62: return aux::wigner_rows<6, 2>(wigner, perm, num_edges, dk, s);
    default: return aux::wigner_rows<6, 6>(wigner, perm, num_edges, dk, s);
  }
}
