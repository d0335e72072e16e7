// Edge-degree embedding (EdgeDegreeEmbedding.forward, reference
// src/maloq/helm/nn/embedding.py:82-141) on gfx950.
//
// The reference pads the radial output u_e [(L+1), C] (one row per degree l,
// the m = 0 coefficients) with zeros to the kept m-major rows, permutes them
// to l-major (einsum with to_m) and rotates back with bmm(wigner_inv).  Only
// the m = 0 column of each block of wigner_inv = D^T meets a non-zero, so the
// per-edge embedding is a rank-one product per degree:
//     emb_e[l^2 + j][c] = D^l_e[l][j] u_e[l][c]            (j = 0 .. 2l)
// (row l of D^l is its m = 0 row).  Node mode then adds emb_e / rescale into
// x[dst_e] (x.index_add_), edge mode returns emb_e in the dtype of x.
//
// No dense product, no float atomics:
//   * the m = 0 rows of D come either from the caller's dense wigner_inv (a
//     column gather, the reference's interface) or straight from the Euler
//     angles with the same recurrence as the dense Wigner kernel (then no
//     [E, d, d] matrix exists at all);
//   * node mode: one workgroup per node (a thread per channel) walks its edges
//     in the dst-sorted, stable order (the order index_add_ adds them in),
//     accumulating in fp32 registers on top of x[node]; deterministic.
#include "message_impl.h"
#include "wigner_device.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace emb {

using msg::static_for;

constexpr int NT = 256;    // threads per workgroup
constexpr int ECH = 32;    // edges per chunk of staged D rows
constexpr int CMAX = 256;  // channels (node mode: one thread per channel)

struct Args {
  const void* u;            // [E, (L+1) C] radial rows (u_bf16 ? bf16 : fp32), original edge order
  int u_bf16;
  int64_t E;
  int C;
  const float* rows;        // [E, d]: rows[e][l^2 + j] = D^l_e[l][j]
  const int64_t* seg_ptr;   // node mode: [N + 1] CSR of the dst-sorted edges
  const int64_t* perm;      // node mode: dst-sorted position -> edge id
  int64_t N;
  float rescale;
  void* x;                  // node mode: [N, d, C] (x_bf16 ? bf16 : fp32), updated in place
  int x_bf16;
  void* edge_out;           // edge mode: [E, d, C] in the dtype of x
};

template <bool BF>
__device__ __forceinline__ float ldt(const void* p, int64_t i) {
  return BF ? bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[i]) : reinterpret_cast<const float*>(p)[i];
}
template <bool BF>
__device__ __forceinline__ void stt(void* p, int64_t i, float v) {
  if constexpr (BF)
    reinterpret_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else
    reinterpret_cast<float*>(p)[i] = v;
}

// Row l (m = 0) of D^l for the static degree l of one edge into out[0 .. 2l]:
// D^l = X(a) J X(b) J X(c) and row l of X(a) is e_l, so the row is
// sum_k J[l][k] M2[k][.] with M2 = X(b) J X(c), summed in the order of the
// dense kernel (wigner_d_row).
template <int l>
__device__ __forceinline__ void m0_row_euler(const float* sJ, float b, float c, float* out) {
  constexpr int n = 2 * l + 1;
  float cb[l + 1], sb[l + 1], cc[l + 1], sc[l + 1];
#pragma unroll
  for (int m = 0; m <= l; ++m) {
    sincos_m(m, b, &sb[m], &cb[m]);
    sincos_m(m, c, &sc[m], &cc[m]);
  }
  const float* J = sJ + jd_offset(l);
  float acc[n], m2[n];
#pragma unroll
  for (int j = 0; j < n; ++j) acc[j] = 0.f;
#pragma unroll
  for (int k = 0; k < n; ++k) {
    wigner_m2_row(l, k, J, cb, sb, cc, sc, m2);
    const float jk = J[l * n + k];
#pragma unroll
    for (int j = 0; j < n; ++j) acc[j] = fmaf(jk, m2[j], acc[j]);
  }
#pragma unroll
  for (int j = 0; j < n; ++j) out[j] = acc[j];
}

// rows[e][l^2 + j] = D^l_e[l][j]: from the dense wigner_inv (its (l^2 + l)-th
// column) or from the Euler angles, thread (edge, static degree l).
template <int L>
__global__ __launch_bounds__(NT) void m0_rows_kernel(const float* __restrict__ wigner_inv,
                                                     const float* __restrict__ eulers,
                                                     const float* __restrict__ jd, int64_t E,
                                                     float* __restrict__ rows) {
  constexpr int d = (L + 1) * (L + 1);
  __shared__ float sJ[jd_size(L)];
  const int tid = threadIdx.x;
  if (wigner_inv != nullptr) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * NT + tid;
    if (i >= E * d) return;
    const int64_t e = i / d;
    const int r = static_cast<int>(i - e * d);
    int l = 0;
    while ((l + 1) * (l + 1) <= r) ++l;
    rows[i] = wigner_inv[e * d * d + static_cast<int64_t>(r) * d + l * l + l];
    return;
  }
  for (int i = tid; i < jd_size(L); i += NT) sJ[i] = jd[i];
  __syncthreads();
  // blockIdx.y = degree l: one degree per launch row keeps each thread's code static
  const int64_t e = static_cast<int64_t>(blockIdx.x) * NT + tid;
  if (e >= E) return;
  const float b = eulers[e * 3 + 1], c = eulers[e * 3 + 2];
  static_for<L + 1>([&](auto LC) {
    constexpr int l = decltype(LC)::value;
    if (static_cast<int>(blockIdx.y) == l) {
      float r[2 * l + 1];
      m0_row_euler<l>(sJ, b, c, r);
#pragma unroll
      for (int j = 0; j <= 2 * l; ++j) rows[e * d + l * l + j] = r[j];
    }
  });
}

// Node mode: workgroup = one node, thread = one channel (blockDim = C rounded
// up to a wave); each thread keeps the node's d outputs of its channel in
// registers (row r of degree l(r), static), walks the node's edges in order,
// four at a time with all their u loads issued together.
template <int L, bool UBF, bool XBF>
__global__ __launch_bounds__(NT) void edge_degree_node_kernel(Args a) {
  constexpr int d = (L + 1) * (L + 1);
  __shared__ float sD[ECH * d];
  __shared__ int64_t sE[ECH];
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t node = blockIdx.x;
  const int64_t s0 = a.seg_ptr[node], s1 = a.seg_ptr[node + 1];
  if (s1 == s0) return;  // no edges: x[node] stays as it is (whole workgroup)
  const int C = a.C;
  const bool live = tid < C;
  const int c = live ? tid : 0;  // idle lanes read channel 0, store nothing
  const int64_t xo = node * d * C + c;
  float acc[d];
#pragma unroll
  for (int r = 0; r < d; ++r) acc[r] = ldt<XBF>(a.x, xo + static_cast<int64_t>(r) * C);
  // the embedding is rounded to the dtype of x (as the reference casts it)
  // and scaled by 1 / rescale (within one rounding of the reference's division)
  const float inv = 1.0f / a.rescale;
  auto add_edge = [&](int e, const float (&uv)[L + 1]) {
#pragma unroll
    for (int l = 0; l <= L; ++l)
#pragma unroll
      for (int j = 0; j <= 2 * l; ++j) {
        float v = sD[e * d + l * l + j] * uv[l];
        if constexpr (XBF) v = bf16_to_f32(f32_to_bf16(v));
        acc[l * l + j] = fmaf(v, inv, acc[l * l + j]);
      }
  };
  for (int64_t c0 = s0; c0 < s1; c0 += ECH) {
    const int ne = static_cast<int>((s1 - c0) < ECH ? (s1 - c0) : ECH);
    __syncthreads();  // previous chunk's rows consumed
    if (tid < ne) sE[tid] = a.perm[c0 + tid];
    __syncthreads();
    for (int i = tid; i < ne * d; i += nt) {
      const int e = i / d;
      sD[i] = a.rows[sE[e] * d + (i - e * d)];
    }
    __syncthreads();
    int e = 0;
    for (; e + 4 <= ne; e += 4) {
      float uv[4][L + 1];
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int l = 0; l <= L; ++l)
          uv[q][l] = ldt<UBF>(a.u, sE[e + q] * static_cast<int64_t>((L + 1) * C) + l * C + c);
#pragma unroll
      for (int q = 0; q < 4; ++q) add_edge(e + q, uv[q]);
    }
    for (; e < ne; ++e) {
      float uv[L + 1];
#pragma unroll
      for (int l = 0; l <= L; ++l) uv[l] = ldt<UBF>(a.u, sE[e] * static_cast<int64_t>((L + 1) * C) + l * C + c);
      add_edge(e, uv);
    }
  }
  if (live) {
#pragma unroll
    for (int r = 0; r < d; ++r) stt<XBF>(a.x, xo + static_cast<int64_t>(r) * C, acc[r]);
  }
}

// Edge mode: out[e][r][c] = rows[e][r] u[e][l(r) C + c] in the dtype of x.
template <int L, bool UBF, bool XBF>
__global__ __launch_bounds__(NT) void edge_degree_edge_kernel(Args a) {
  constexpr int d = (L + 1) * (L + 1);
  const int C = a.C;
  const int64_t n = a.E * d * C;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x; o < n;
       o += static_cast<int64_t>(gridDim.x) * NT) {
    const int64_t e = o / (d * C);
    const int rc = static_cast<int>(o - e * d * C);
    const int r = rc / C, c = rc - (rc / C) * C;
    int l = 0;
    while ((l + 1) * (l + 1) <= r) ++l;
    stt<XBF>(a.edge_out, o, a.rows[e * d + r] * ldt<UBF>(a.u, e * (L + 1) * C + l * C + c));
  }
}

// Backward with respect to u: grad_u[e][l C + c] = scale sum_j D^l_e[l][j]
// g[row_e][l^2 + j][c], row_e = dst_e (node mode, through index_add_) or e
// (edge mode), j ascending.
template <int L, bool GBF>
__global__ __launch_bounds__(NT) void edge_degree_bwd_kernel(const void* __restrict__ g,
                                                             const int64_t* __restrict__ grow,
                                                             const float* __restrict__ rows, int64_t E,
                                                             int C, float scale, float* __restrict__ grad_u) {
  constexpr int d = (L + 1) * (L + 1);
  const int64_t n = E * (L + 1) * C;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * NT + threadIdx.x; o < n;
       o += static_cast<int64_t>(gridDim.x) * NT) {
    const int64_t e = o / ((L + 1) * C);
    const int lc = static_cast<int>(o - e * (L + 1) * C);
    const int l = lc / C, c = lc - (lc / C) * C;
    const int64_t go = (grow != nullptr ? grow[e] : e) * d * C + static_cast<int64_t>(l * l) * C + c;
    float acc = 0.f;
    for (int j = 0; j <= 2 * l; ++j) acc = fmaf(rows[e * d + l * l + j], ldt<GBF>(g, go + static_cast<int64_t>(j) * C), acc);
    grad_u[o] = acc * scale;
  }
}

static unsigned blocks_for(int64_t n) {
  const int64_t b = (n + NT - 1) / NT;
  return static_cast<unsigned>(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

template <int L>
static void launch_rows(const float* wigner_inv, const float* eulers, const float* jd, int64_t E, float* rows,
                        hipStream_t s) {
  constexpr int d = (L + 1) * (L + 1);
  if (wigner_inv != nullptr)
    hipLaunchKernelGGL(m0_rows_kernel<L>, dim3(static_cast<unsigned>((E * d + NT - 1) / NT)), dim3(NT), 0, s,
                       wigner_inv, eulers, jd, E, rows);
  else
    hipLaunchKernelGGL(m0_rows_kernel<L>, dim3(static_cast<unsigned>((E + NT - 1) / NT), L + 1), dim3(NT), 0, s,
                       wigner_inv, eulers, jd, E, rows);
}

template <int L, bool UBF, bool XBF>
static void launch_embed(const Args& a, hipStream_t s) {
  if (a.edge_out != nullptr)
    hipLaunchKernelGGL((edge_degree_edge_kernel<L, UBF, XBF>),
                       dim3(blocks_for(a.E * (L + 1) * (L + 1) * a.C)), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL((edge_degree_node_kernel<L, UBF, XBF>), dim3(static_cast<unsigned>(a.N)),
                       dim3(static_cast<unsigned>((a.C + 63) / 64 * 64)), 0, s, a);
}

template <int L>
static void launch(const Args& a, hipStream_t s) {
  if (a.u_bf16 && a.x_bf16)
    launch_embed<L, true, true>(a, s);
  else if (a.u_bf16)
    launch_embed<L, true, false>(a, s);
  else if (a.x_bf16)
    launch_embed<L, false, true>(a, s);
  else
    launch_embed<L, false, false>(a, s);
}

template <int L>
static void launch_bwd(int g_bf16, const void* g, const int64_t* grow, const float* rows, int64_t E, int C,
                       float scale, float* grad_u, hipStream_t s) {
  const dim3 grid(blocks_for(E * (L + 1) * C));
  if (g_bf16)
    hipLaunchKernelGGL((edge_degree_bwd_kernel<L, true>), grid, dim3(NT), 0, s, g, grow, rows, E, C, scale, grad_u);
  else
    hipLaunchKernelGGL((edge_degree_bwd_kernel<L, false>), grid, dim3(NT), 0, s, g, grow, rows, E, C, scale, grad_u);
}

}  // namespace emb
}  // namespace maloq

using namespace maloq;

#define MALOQ_EMB_SWITCH(LMAX, CALL)  \
  switch (LMAX) {                     \
    case 0: CALL(0); break;           \
    case 1: CALL(1); break;           \
    case 2: CALL(2); break;           \
    case 3: CALL(3); break;           \
    case 4: CALL(4); break;           \
    case 5: CALL(5); break;           \
    default: CALL(6); break;          \
  }

extern "C" int maloq_edge_m0_rows(int lmax, int64_t num_edges, const float* wigner_inv, const float* eulers,
                                  const float* jd, float* rows, void* stream) {
  MALOQ_REQUIRE(lmax >= 0 && lmax <= 6, "lmax must be 0-6, got %d", lmax);
  MALOQ_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 31), "edge count out of range");
  if (num_edges == 0) return MALOQ_OK;
  MALOQ_REQUIRE((wigner_inv != nullptr) != (eulers != nullptr), "give exactly one of wigner_inv, eulers");
  MALOQ_REQUIRE(eulers == nullptr || jd != nullptr, "jd is null");
  MALOQ_REQUIRE(rows != nullptr, "rows is null");
  hipStream_t s = static_cast<hipStream_t>(stream);
#define MALOQ_EMB_ROWS(L) emb::launch_rows<L>(wigner_inv, eulers, jd, num_edges, rows, s)
  MALOQ_EMB_SWITCH(lmax, MALOQ_EMB_ROWS)
#undef MALOQ_EMB_ROWS
  return check_launch("m0_rows_kernel");
}

extern "C" int maloq_edge_degree_embed(int u_dtype, int x_dtype, int lmax, const void* u, int64_t num_edges,
                                       int channels, const float* rows, const int64_t* seg_ptr,
                                       const int64_t* perm, int64_t num_nodes, float rescale, void* x,
                                       void* edge_out, void* stream) {
  MALOQ_REQUIRE(u_dtype == 0 || u_dtype == 1, "u dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(x_dtype == 0 || x_dtype == 1, "x dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(lmax >= 0 && lmax <= 6, "lmax must be 0-6, got %d", lmax);
  MALOQ_REQUIRE(channels > 0 && channels <= emb::CMAX, "channels must be 1-%d", emb::CMAX);
  MALOQ_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 31), "edge count out of range");
  MALOQ_REQUIRE(num_nodes >= 0 && num_nodes < (int64_t(1) << 31), "node count out of range");
  MALOQ_REQUIRE(rescale != 0.f, "rescale is zero");
  if (num_edges == 0 || (edge_out == nullptr && num_nodes == 0)) return MALOQ_OK;  // nothing to add
  MALOQ_REQUIRE(u != nullptr && rows != nullptr, "null pointer");
  if (edge_out == nullptr) MALOQ_REQUIRE(seg_ptr && perm && x, "null pointer");
  emb::Args a{};
  a.u = u;
  a.u_bf16 = u_dtype;
  a.E = num_edges;
  a.C = channels;
  a.rows = rows;
  a.seg_ptr = seg_ptr;
  a.perm = perm;
  a.N = num_nodes;
  a.rescale = rescale;
  a.x = x;
  a.x_bf16 = x_dtype;
  a.edge_out = edge_out;
  hipStream_t s = static_cast<hipStream_t>(stream);
#define MALOQ_EMB_FWD(L) emb::launch<L>(a, s)
  MALOQ_EMB_SWITCH(lmax, MALOQ_EMB_FWD)
#undef MALOQ_EMB_FWD
  return check_launch("edge_degree_kernel");
}

extern "C" int maloq_edge_degree_embed_bwd(int g_dtype, int lmax, const void* grad, const int64_t* grad_rows,
                                           int64_t num_edges, int channels, const float* rows, float scale,
                                           float* grad_u, void* stream) {
  MALOQ_REQUIRE(g_dtype == 0 || g_dtype == 1, "grad dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(lmax >= 0 && lmax <= 6, "lmax must be 0-6, got %d", lmax);
  MALOQ_REQUIRE(channels > 0 && channels <= emb::CMAX, "channels must be 1-%d", emb::CMAX);
  MALOQ_REQUIRE(num_edges >= 0 && num_edges < (int64_t(1) << 31), "edge count out of range");
  if (num_edges == 0) return MALOQ_OK;
  MALOQ_REQUIRE(grad && rows && grad_u, "null pointer");
  hipStream_t s = static_cast<hipStream_t>(stream);
#define MALOQ_EMB_BWD(L) emb::launch_bwd<L>(g_dtype, grad, grad_rows, rows, num_edges, channels, scale, grad_u, s)
  MALOQ_EMB_SWITCH(lmax, MALOQ_EMB_BWD)
#undef MALOQ_EMB_BWD
  return check_launch("edge_degree_bwd_kernel");
}
