// Elementwise stages of the Fock irreps output head (gfx950): the gated
// nonlinearity between the head's two linear maps, and the column gather that
// puts the per-l outputs in label order (and expands the reduced node irreps).
//
// Reference: Fock_Irreps_Head.process / forward / expand_reduced_node
// (helm/esen_osh.py:894-1052, 1055-1064).  With x the backbone features
// [B, d, C] (d = (L+1)^2, rows l-major as the backbone keeps them, so the
// reference's stack_irreps reorder is never materialised) and s = the scalar
// linear's output [B, C + L C]:
//   g[b, 0, c]        = s[b, c]                                   (transformed l = 0)
//   g[b, l^2 + m, c]  = cst sigmoid(s[b, C + (l-1) C + c]) x[b, l^2 + m, c]   (l >= 1)
// (e3nn's Gate with normalised activation: cst = E[sigmoid(z)^2]^-1/2, z ~ N(0,1)).
// With reduce_edge the gate must keep odd data odd: the activation is then
// cst tanh(|s|) (e3nn's Gate with tanh gates on |gating scalars|, :994-995),
// selected by act = 1; act = 0 is cst sigmoid(s).
// The labels are then out[r, t] = sign[t] in[r, src[t]] (0 where src[t] < 0),
// and the gradient of that gather is a fixed-order sum over the columns that
// read each input column (CSR), so it is deterministic without atomics.
#include "common.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace ih {

__device__ __forceinline__ float sigmoidf(float z) { return 1.0f / (1.0f + expf(-z)); }

// The gate activation f(z) and f'(z): sigmoid (act 0), or tanh(|z|) (act 1)
// with d|z|/dz = sign(z), 0 at z = 0 (as torch's abs).
__device__ __forceinline__ float gate_act(int act, float z) { return act ? tanhf(fabsf(z)) : sigmoidf(z); }
__device__ __forceinline__ float gate_dact(int act, float z, float f) {
  if (act) return (1.0f - f * f) * (z > 0.f ? 1.0f : (z < 0.f ? -1.0f : 0.f));
  return f * (1.0f - f);
}

// One thread per (b, row, channel); consecutive threads take consecutive channels.
__global__ void gate_fwd_kernel(const float* __restrict__ x, int64_t B, int L, int C, const float* __restrict__ s,
                                float cst, int act, float* __restrict__ g) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int d = (L + 1) * (L + 1);
  if (i >= B * d * C) return;
  const int64_t b = i / (static_cast<int64_t>(d) * C);
  const int rem = static_cast<int>(i - b * d * C);
  const int j = rem / C, c = rem - j * C;
  const float* sb = s + b * (C + static_cast<int64_t>(L) * C);
  if (j == 0) {
    g[i] = sb[c];
    return;
  }
  int l = 1;  // degree of row j: l^2 <= j < (l+1)^2
  while ((l + 1) * (l + 1) <= j) ++l;
  g[i] = cst * gate_act(act, sb[C + (l - 1) * C + c]) * x[i];
}

// The same with one thread per (b, 4 channels) over the d rows (C % 4 == 0,
// 16-byte aligned arrays): each degree's gate factors are evaluated once, the
// rows are 16-byte loads and stores, consecutive threads take consecutive
// channel groups.  Same products as gate_fwd_kernel, so the same bits.
__global__ void gate_fwd4_kernel(const float* __restrict__ x, int64_t B, int L, int C, const float* __restrict__ s,
                                 float cst, int act, float* __restrict__ g) {
  const int C4 = C >> 2;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= B * C4) return;
  const int64_t b = i / C4;
  const int c = static_cast<int>(i - b * C4) * 4;
  const int d = (L + 1) * (L + 1);
  const float* sb = s + b * (C + static_cast<int64_t>(L) * C);
  const float4* xb = reinterpret_cast<const float4*>(x + b * d * C + c);
  float4* gb = reinterpret_cast<float4*>(g + b * d * C + c);
  gb[0] = *reinterpret_cast<const float4*>(sb + c);
  for (int l = 1; l <= L; ++l) {
    const float4 z = *reinterpret_cast<const float4*>(sb + C + (l - 1) * C + c);
    const float4 f = make_float4(cst * gate_act(act, z.x), cst * gate_act(act, z.y), cst * gate_act(act, z.z),
                                 cst * gate_act(act, z.w));
    for (int j = l * l; j < (l + 1) * (l + 1); ++j) {
      const float4 v = xb[static_cast<int64_t>(j) * C4];
      gb[static_cast<int64_t>(j) * C4] = make_float4(f.x * v.x, f.y * v.y, f.z * v.z, f.w * v.w);
    }
  }
}

// One thread per (b, channel): the d rows of that channel.
//   dx[b, l^2 + m, c]           = go g_l          (l >= 1; row 0 untouched: x's l = 0
//                                                 only feeds the scalar linear)
//   ds[b, c]                    = go[b, 0, c]
//   ds[b, C + (l-1) C + c]      = cst f'(z) sum_m go[b, l^2 + m, c] x[b, l^2 + m, c]
__global__ void gate_bwd_kernel(const float* __restrict__ x, int64_t B, int L, int C, const float* __restrict__ s,
                                float cst, int act, const float* __restrict__ go, float* __restrict__ dx,
                                float* __restrict__ ds) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= B * C) return;
  const int64_t b = i / C;
  const int c = static_cast<int>(i - b * C);
  const int d = (L + 1) * (L + 1);
  const int64_t ws = C + static_cast<int64_t>(L) * C;
  const float* sb = s + b * ws;
  float* dsb = ds + b * ws;
  const int64_t rb = b * static_cast<int64_t>(d) * C + c;
  dsb[c] = go[rb];
  dx[rb] = 0.f;
  for (int l = 1; l <= L; ++l) {
    const float z = sb[C + (l - 1) * C + c];
    const float sg = gate_act(act, z);
    const float gl = cst * sg;
    float acc = 0.f;
    for (int m = 0; m < 2 * l + 1; ++m) {
      const int64_t k = rb + static_cast<int64_t>(l * l + m) * C;
      const float gv = go[k];
      acc = fmaf(gv, x[k], acc);
      dx[k] = gv * gl;
    }
    dsb[C + (l - 1) * C + c] = acc * cst * gate_dact(act, z, sg);
  }
}

// out[r, t] = src[t] >= 0 ? sign[t] in[r, src[t]] : 0; a thread per (r, t).
__global__ void gather_cols_kernel(const float* __restrict__ in, int64_t ld_in, int64_t R,
                                   const int32_t* __restrict__ src, const float* __restrict__ sign, int T,
                                   float* __restrict__ out, int64_t ld_out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= R * T) return;
  const int64_t r = i / T;
  const int t = static_cast<int>(i - r * T);
  const int sc = src[t];
  out[r * ld_out + t] = sc >= 0 ? sign[t] * in[r * ld_in + sc] : 0.f;
}

// din[r, s] = sum_{k in [ptr[s], ptr[s+1])} sign[k] dout[r, col[k]] in k order; a thread per (r, s).
__global__ void scatter_cols_kernel(const float* __restrict__ dout, int64_t ld_out, int64_t R,
                                    const int32_t* __restrict__ ptr, const int32_t* __restrict__ col,
                                    const float* __restrict__ sign, int S, float* __restrict__ din, int64_t ld_in) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= R * S) return;
  const int64_t r = i / S;
  const int sc = static_cast<int>(i - r * S);
  float acc = 0.f;
  for (int k = ptr[sc]; k < ptr[sc + 1]; ++k) acc = fmaf(sign[k], dout[r * ld_out + col[k]], acc);
  din[r * ld_in + sc] = acc;
}

int grid_of(int64_t n, unsigned* g) {
  const int64_t blocks = (n + 255) / 256;
  MALOQ_REQUIRE(blocks < (int64_t(1) << 31), "grid too large");
  *g = static_cast<unsigned>(blocks);
  return MALOQ_OK;
}

}  // namespace ih
}  // namespace maloq

using namespace maloq;

extern "C" int maloq_irreps_gate_fwd(const float* x, int64_t num_rows, int lmax, int c, const float* scalars, float cst,
                                     int act, float* out, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && lmax >= 0 && lmax <= 8 && c > 0, "bad sizes");
  MALOQ_REQUIRE(act == 0 || act == 1, "act must be 0 (sigmoid) or 1 (tanh of |z|)");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(x && scalars && out && out != x, "null or aliased pointer");
  const int d = (lmax + 1) * (lmax + 1);
  unsigned g;
  const bool v4 = c % 4 == 0 && ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(scalars) |
                                  reinterpret_cast<uintptr_t>(out)) & 15) == 0;
  if (v4) {
    if (ih::grid_of(num_rows * (c / 4), &g)) return MALOQ_EINVAL;
    hipLaunchKernelGGL(ih::gate_fwd4_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), x, num_rows,
                       lmax, c, scalars, cst, act, out);
    return check_launch("gate_fwd4_kernel");
  }
  if (ih::grid_of(num_rows * d * c, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(ih::gate_fwd_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), x, num_rows, lmax,
                     c, scalars, cst, act, out);
  return check_launch("gate_fwd_kernel");
}

extern "C" int maloq_irreps_gate_bwd(const float* x, int64_t num_rows, int lmax, int c, const float* scalars, float cst,
                                     int act, const float* grad_out, float* grad_x, float* grad_scalars,
                                     void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && lmax >= 0 && lmax <= 8 && c > 0, "bad sizes");
  MALOQ_REQUIRE(act == 0 || act == 1, "act must be 0 (sigmoid) or 1 (tanh of |z|)");
  if (num_rows == 0) return MALOQ_OK;
  MALOQ_REQUIRE(x && scalars && grad_out && grad_x && grad_scalars, "null pointer");
  unsigned g;
  if (ih::grid_of(num_rows * c, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(ih::gate_bwd_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), x, num_rows, lmax,
                     c, scalars, cst, act, grad_out, grad_x, grad_scalars);
  return check_launch("gate_bwd_kernel");
}

extern "C" int maloq_gather_columns(const float* in, int64_t ld_in, int64_t num_rows, const int32_t* src,
                                    const float* sign, int t, float* out, int64_t ld_out, void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && t >= 0 && ld_out >= t, "bad sizes");
  if (num_rows == 0 || t == 0) return MALOQ_OK;
  MALOQ_REQUIRE(in && src && sign && out && in != out, "null or aliased pointer");
  unsigned g;
  if (ih::grid_of(num_rows * t, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(ih::gather_cols_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), in, ld_in,
                     num_rows, src, sign, t, out, ld_out);
  return check_launch("gather_cols_kernel");
}

extern "C" int maloq_scatter_columns(const float* grad_out, int64_t ld_out, int64_t num_rows, const int32_t* ptr,
                                     const int32_t* cols, const float* sign, int s, float* grad_in, int64_t ld_in,
                                     void* stream) {
  MALOQ_REQUIRE(num_rows >= 0 && s >= 0 && ld_in >= s, "bad sizes");
  if (num_rows == 0 || s == 0) return MALOQ_OK;
  MALOQ_REQUIRE(grad_out && ptr && cols && sign && grad_in && grad_out != grad_in, "null or aliased pointer");
  unsigned g;
  if (ih::grid_of(num_rows * s, &g)) return MALOQ_EINVAL;
  hipLaunchKernelGGL(ih::scatter_cols_kernel, dim3(g), dim3(256), 0, static_cast<hipStream_t>(stream), grad_out,
                     ld_out, num_rows, ptr, cols, sign, s, grad_in, ld_in);
  return check_launch("scatter_cols_kernel");
}
