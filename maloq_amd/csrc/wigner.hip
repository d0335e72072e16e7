// Per-edge Euler angles and dense block-diagonal Wigner-D matrices (gfx950).
//
// Replaces the reference's Triton kernels wigner_fused_kernel_16/_32 and
// _extract_eulers_kernel (src/maloq/helm/triton_kernels/wigner_fused.py:150-380).
// One workgroup handles a batch of edges; each thread owns one output row of
// one edge: it builds row k of X(b) J X(c) into LDS, then row i of D_l, and the
// batch's [E_b, d, d] slab (and optionally its transpose) is written with
// coalesced stores.
#include "common.h"
#include "wigner_device.h"
#include "../../include/maloq_hip.h"

namespace maloq {

template <int L>
struct WignerShape {
  static constexpr int d = (L + 1) * (L + 1);
  static constexpr int EPB = (256 / d) > 0 ? (256 / d) : 1;  // edges per block
  static constexpr int JSZ = jd_size(L);
};

template <int L>
__global__ __launch_bounds__(256) void wigner_dense_kernel(
    const float* __restrict__ vec, const float* __restrict__ eulers_in, uint64_t seed,
    int64_t num_edges, const float* __restrict__ jd, float* __restrict__ eulers_out,
    float* __restrict__ out, float* __restrict__ out_inv, int write_zeros) {
  using S = WignerShape<L>;
  constexpr int d = S::d, EPB = S::EPB, JSZ = S::JSZ;
  __shared__ float sJ[JSZ];
  __shared__ float sTrig[EPB][3][2][L + 1];  // [edge][angle a,b,c][cos,sin][m]
  __shared__ float sM2[EPB][JSZ];
  __shared__ float sD[EPB][JSZ];

  const int t = threadIdx.x;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * EPB;
  for (int i = t; i < JSZ; i += blockDim.x) sJ[i] = jd[i];

  const int el = t / d;
  const int row = t - el * d;
  const int64_t e = e0 + el;
  const bool active = (el < EPB) && (e < num_edges);
  int l = 0;
  while ((l + 1) * (l + 1) <= row) ++l;
  const int i = row - l * l;

  // Angles: one thread per edge computes them (or reads them).
  __shared__ float sAng[EPB][3];
  if (active && row == 0) {
    float a, b, c;
    if (eulers_in != nullptr) {
      a = eulers_in[e * 3 + 0];
      b = eulers_in[e * 3 + 1];
      c = eulers_in[e * 3 + 2];
    } else {
      edge_euler(vec[e * 3 + 0], vec[e * 3 + 1], vec[e * 3 + 2], philox_uniform(seed, e), &a, &b,
                 &c);
      if (eulers_out != nullptr) {
        eulers_out[e * 3 + 0] = a;
        eulers_out[e * 3 + 1] = b;
        eulers_out[e * 3 + 2] = c;
      }
    }
    sAng[el][0] = a;
    sAng[el][1] = b;
    sAng[el][2] = c;
  }
  __syncthreads();
  if (active) {
    for (int q = row; q < 3 * (L + 1); q += d) {
      const int ang = q / (L + 1), m = q - ang * (L + 1);
      float s, c;
      sincos_m(m, sAng[el][ang], &s, &c);
      sTrig[el][ang][0][m] = c;
      sTrig[el][ang][1][m] = s;
    }
  }
  __syncthreads();
  const int jo = (l == 0) ? 0 : jd_offset(l);
  const int n = 2 * l + 1;
  if (active) {
    wigner_m2_row(l, i, sJ + jo, sTrig[el][1][0], sTrig[el][1][1], sTrig[el][2][0],
                  sTrig[el][2][1], &sM2[el][jo + i * n]);
  }
  __syncthreads();
  if (active) {
    wigner_d_row(l, i, sJ + jo, &sM2[el][jo], sTrig[el][0][0], sTrig[el][0][1],
                 &sD[el][jo + i * n]);
  }
  __syncthreads();

  // Coalesced write of the batch slab.
  const int64_t nvalid = (num_edges - e0) < EPB ? (num_edges - e0) : EPB;
  const int64_t total = nvalid * d * d;
  float* o = out + e0 * d * d;
  float* oi = out_inv ? out_inv + e0 * d * d : nullptr;
  for (int64_t idx = t; idx < total; idx += blockDim.x) {
    const int eb = static_cast<int>(idx / (d * d));
    const int rc = static_cast<int>(idx - static_cast<int64_t>(eb) * d * d);
    const int r = rc / d, c = rc - r * d;
    int lr = 0;
    while ((lr + 1) * (lr + 1) <= r) ++lr;
    const bool in_block = (c >= lr * lr) && (c < (lr + 1) * (lr + 1));
    if (in_block) {
      const int nb = 2 * lr + 1, off = (lr == 0) ? 0 : jd_offset(lr);
      const int ri = r - lr * lr, ci = c - lr * lr;
      if (o) o[idx] = sD[eb][off + ri * nb + ci];
      if (oi) oi[idx] = sD[eb][off + ci * nb + ri];
    } else if (write_zeros) {
      if (o) o[idx] = 0.0f;
      if (oi) oi[idx] = 0.0f;
    }
  }
}

__global__ void euler_kernel(const float* __restrict__ vec, uint64_t seed, int64_t num_edges,
                             float* __restrict__ eulers) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= num_edges) return;
  float a, b, c;
  edge_euler(vec[e * 3 + 0], vec[e * 3 + 1], vec[e * 3 + 2], philox_uniform(seed, e), &a, &b, &c);
  eulers[e * 3 + 0] = a;
  eulers[e * 3 + 1] = b;
  eulers[e * 3 + 2] = c;
}

template <int L>
static void launch_dense(const float* vec, const float* eulers_in, uint64_t seed, int64_t E,
                         const float* jd, float* eulers_out, float* out, float* out_inv,
                         int write_zeros, hipStream_t s) {
  using S = WignerShape<L>;
  const int64_t blocks = (E + S::EPB - 1) / S::EPB;
  hipLaunchKernelGGL(wigner_dense_kernel<L>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                     vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros);
}

static int dense_dispatch(const float* vec, const float* eulers_in, uint64_t seed, int64_t E,
                          int lmax, const float* jd, float* eulers_out, float* out, float* out_inv,
                          int write_zeros, hipStream_t s) {
  MALOQ_REQUIRE(lmax >= 0 && lmax <= 8, "lmax must be 0-8, got %d", lmax);
  MALOQ_REQUIRE(E >= 0, "num_edges must be >= 0");
  if (E == 0) return MALOQ_OK;
  MALOQ_REQUIRE(jd != nullptr, "jd is null");
  MALOQ_REQUIRE(out != nullptr || out_inv != nullptr, "no output given");
  MALOQ_REQUIRE(E < (int64_t(1) << 31), "too many edges");
  switch (lmax) {
    case 0: launch_dense<0>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 1: launch_dense<1>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 2: launch_dense<2>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 3: launch_dense<3>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 4: launch_dense<4>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 5: launch_dense<5>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 6: launch_dense<6>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    case 7: launch_dense<7>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
    default: launch_dense<8>(vec, eulers_in, seed, E, jd, eulers_out, out, out_inv, write_zeros, s); break;
  }
  return check_launch("wigner_dense_kernel");
}

}  // namespace maloq

extern "C" int maloq_edge_euler(const float* edge_vec, int64_t num_edges, uint64_t seed,
                                float* eulers, void* stream) {
  MALOQ_REQUIRE(num_edges >= 0, "num_edges must be >= 0");
  if (num_edges == 0) return MALOQ_OK;
  MALOQ_REQUIRE(edge_vec && eulers, "null pointer");
  const int64_t blocks = (num_edges + 255) / 256;
  hipLaunchKernelGGL(maloq::euler_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), edge_vec, seed, num_edges, eulers);
  return maloq::check_launch("euler_kernel");
}

extern "C" int maloq_edge_vec_to_wigner(const float* edge_vec, int64_t num_edges, uint64_t seed,
                                        int lmax, const float* jd_packed, float* eulers_out,
                                        float* wigner, float* wigner_inv, int write_zeros,
                                        void* stream) {
  if (num_edges > 0) MALOQ_REQUIRE(edge_vec != nullptr, "edge_vec is null");
  return maloq::dense_dispatch(edge_vec, nullptr, seed, num_edges, lmax, jd_packed, eulers_out,
                               wigner, wigner_inv, write_zeros, static_cast<hipStream_t>(stream));
}

extern "C" int maloq_wigner_from_euler(const float* eulers, int64_t num_edges, int lmax,
                                       const float* jd_packed, float* wigner, float* wigner_inv,
                                       int write_zeros, void* stream) {
  if (num_edges > 0) MALOQ_REQUIRE(eulers != nullptr, "eulers is null");
  return maloq::dense_dispatch(nullptr, eulers, 0, num_edges, lmax, jd_packed, nullptr, wigner,
                               wigner_inv, write_zeros, static_cast<hipStream_t>(stream));
}
