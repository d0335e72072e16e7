// Standalone rotation of irreps features into and out of the edge frame (gfx950).
//
// Replaces the reference's torch.bmm(wigner, x_message) and
// torch.bmm(wigner_inv, x_message) (helm/esen_block.py:181,191 and the heads,
// helm/esen_osh.py:1218,1228,1318,1328) for callers that need the rotated rows
// themselves rather than the fused message block:
//   out[e] = D_e x[g(e)]      (forward: into the edge frame)
//   out[e] = D_e^T x[g(e)]    (inverse: back to the global frame)
// with D_e the block-diagonal Wigner-D of edge e, g(e) = gather[e] (or e).
// D_e comes from the edge's Euler triple (the same recurrence as the dense
// Wigner kernel, so the result equals bmm with that kernel's D) or from the
// block-diagonal part of a caller's dense [E, d, d] wigner; only the
// (2l+1) x (2l+1) blocks are touched: sum_l (2l+1)^2 MACs per channel instead
// of the d^2 of a dense bmm.
//
// A workgroup takes epb <= EPB = 256 / d edges: phase 1 puts their D blocks in
// LDS (one thread per (edge, row), as the dense Wigner kernel); phase 2 runs
// one thread per (edge, 4 channels), reading each degree's 2l+1 input rows as
// 16-byte (fp32) or 8-byte (bf16) vectors and writing the 2l+1 output rows.
// epb = min(EPB, 256 / (C / 4)): phase 2 is then one round of the 256 threads
// (C = 128, d = 25: 8 edges x 32 channel quads) instead of a full round and a
// quarter-wave tail.
// HBM-bound: d C (s_in + s_out) bytes per edge plus 12 (Euler triple).
#include "common.h"
#include "wigner_device.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace rot {

struct Args {
  const void* x;          // [*, d, C]
  const int32_t* gather;  // [E] nullable
  int64_t E;
  int C;
  const float* eulers;    // [E, 3] or null
  const float* wigner;    // [E, d, d] or null
  const float* jd;        // packed J_0..J_L (with eulers)
  int inverse;
  int epb;                // edges per workgroup (<= Shape::EPB)
  void* out;              // [E, d, C]
};

template <int L>
struct Shape {
  static constexpr int d = (L + 1) * (L + 1);
  static constexpr int EPB = (256 / d) > 0 ? (256 / d) : 1;
  static constexpr int JSZ = jd_size(L);
};

__device__ __forceinline__ void load4(const float* p, float (&v)[4]) {
  const float4 t = *reinterpret_cast<const float4*>(p);
  v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
}
__device__ __forceinline__ void load4(const uint16_t* p, float (&v)[4]) {
  const uint2 t = *reinterpret_cast<const uint2*>(p);
  v[0] = __uint_as_float(t.x << 16);
  v[1] = __uint_as_float(t.x & 0xffff0000u);
  v[2] = __uint_as_float(t.y << 16);
  v[3] = __uint_as_float(t.y & 0xffff0000u);
}
__device__ __forceinline__ void store4(float* p, const float (&v)[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store4(uint16_t* p, const float (&v)[4]) {
  uint2 t;
  t.x = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  t.y = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
  *reinterpret_cast<uint2*>(p) = t;
}

template <int L, class TX, class TO>
__global__ __launch_bounds__(256) void rotate_kernel(Args a) {
  using S = Shape<L>;
  constexpr int d = S::d, EPB = S::EPB, JSZ = S::JSZ;
  __shared__ float sJ[JSZ];
  __shared__ float sAng[EPB][3];
  __shared__ float sTrig[EPB][3][2][L + 1];  // [edge][angle a, b, c][cos, sin][m]
  __shared__ float sM2[EPB][JSZ];
  __shared__ float sD[EPB][JSZ];
  const int t = threadIdx.x;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * a.epb;
  const int nvalid = static_cast<int>((a.E - e0) < a.epb ? (a.E - e0) : a.epb);

  // ---- phase 1: the D blocks of the workgroup's edges
  const int el = t / d, row = t - (t / d) * d;
  const bool active = el < nvalid;
  int l = 0;
  while ((l + 1) * (l + 1) <= row) ++l;
  const int i = row - l * l, n = 2 * l + 1, jo = jd_offset(l);
  const int64_t e = e0 + el;
  if (a.wigner != nullptr) {
    if (active) {
      const float* w = a.wigner + (e * d + row) * d + l * l;
      for (int j = 0; j < n; ++j) sD[el][jo + i * n + j] = w[j];
    }
  } else {
    for (int k = t; k < JSZ; k += blockDim.x) sJ[k] = a.jd[k];
    if (active && row == 0) {
      sAng[el][0] = a.eulers[e * 3 + 0];
      sAng[el][1] = a.eulers[e * 3 + 1];
      sAng[el][2] = a.eulers[e * 3 + 2];
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
    if (active)
      wigner_m2_row(l, i, sJ + jo, sTrig[el][1][0], sTrig[el][1][1], sTrig[el][2][0], sTrig[el][2][1],
                    &sM2[el][jo + i * n]);
    __syncthreads();
    if (active) wigner_d_row(l, i, sJ + jo, &sM2[el][jo], sTrig[el][0][0], sTrig[el][0][1], &sD[el][jo + i * n]);
  }
  __syncthreads();

  // ---- phase 2: one thread per (edge, 4 channels)
  const int nch = a.C / 4;
  const typename TX::raw* x = static_cast<const typename TX::raw*>(a.x);
  typename TO::raw* out = static_cast<typename TO::raw*>(a.out);
  for (int u = t; u < nvalid * nch; u += blockDim.x) {
    const int eb = u / nch, c0 = (u - eb * nch) * 4;
    const int64_t ee = e0 + eb;
    const int64_t g = a.gather != nullptr ? a.gather[ee] : ee;
    const typename TX::raw* xr = x + g * d * a.C + c0;
    typename TO::raw* orow = out + ee * d * a.C + c0;
    const float* D = sD[eb];
#pragma unroll
    for (int ll = 0; ll <= L; ++ll) {
      constexpr int NMAX = 2 * L + 1;
      const int nl = 2 * ll + 1, off = jd_offset(ll);
      float xv[NMAX][4];
#pragma unroll
      for (int j = 0; j < NMAX; ++j)
        if (j < nl) load4(xr + (ll * ll + j) * a.C, xv[j]);
#pragma unroll
      for (int r = 0; r < NMAX; ++r) {
        if (r >= nl) break;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NMAX; ++j) {
          if (j >= nl) break;
          const float w = a.inverse ? D[off + j * nl + r] : D[off + r * nl + j];
#pragma unroll
          for (int c = 0; c < 4; ++c) o[c] = fmaf(w, xv[j][c], o[c]);
        }
        store4(orow + (ll * ll + r) * a.C, o);
      }
    }
  }
}

struct F32T {
  using raw = float;
};
struct BF16T {
  using raw = uint16_t;
};

template <int L>
int launch(int x_dtype, int out_dtype, Args a, hipStream_t s) {
  const int by_channels = 256 / (a.C / 4);
  a.epb = by_channels < 1 ? 1 : (by_channels < Shape<L>::EPB ? by_channels : Shape<L>::EPB);
  const int64_t grid = (a.E + a.epb - 1) / a.epb;
  MALOQ_REQUIRE(grid < (int64_t(1) << 31), "grid too large");
  const dim3 g(static_cast<unsigned>(grid)), b(256);
  if (x_dtype == 0 && out_dtype == 0) hipLaunchKernelGGL((rotate_kernel<L, F32T, F32T>), g, b, 0, s, a);
  else if (x_dtype == 1 && out_dtype == 1) hipLaunchKernelGGL((rotate_kernel<L, BF16T, BF16T>), g, b, 0, s, a);
  else if (x_dtype == 1 && out_dtype == 0) hipLaunchKernelGGL((rotate_kernel<L, BF16T, F32T>), g, b, 0, s, a);
  else hipLaunchKernelGGL((rotate_kernel<L, F32T, BF16T>), g, b, 0, s, a);
  return check_launch("rotate_kernel");
}

}  // namespace rot
}  // namespace maloq

using namespace maloq;

extern "C" int maloq_rotate(int x_dtype, int out_dtype, int lmax, const void* x, int c,
                            const int32_t* gather, int64_t num_edges, const float* eulers,
                            const float* wigner, const float* jd, int inverse, void* out,
                            void* stream) {
  MALOQ_REQUIRE((x_dtype == 0 || x_dtype == 1) && (out_dtype == 0 || out_dtype == 1), "dtype must be 0 or 1");
  MALOQ_REQUIRE(lmax >= 0 && lmax <= 8, "lmax must be 0-8, got %d", lmax);
  MALOQ_REQUIRE(c > 0 && c % 4 == 0, "channels must be a positive multiple of 4");
  MALOQ_REQUIRE(num_edges >= 0, "num_edges < 0");
  if (num_edges == 0) return MALOQ_OK;
  MALOQ_REQUIRE(x && out, "null pointer");
  MALOQ_REQUIRE((eulers != nullptr) != (wigner != nullptr), "give exactly one of eulers and wigner");
  MALOQ_REQUIRE(wigner || jd, "the Euler path needs the packed J tables");
  const uintptr_t al = (x_dtype == 0 ? 15 : 7);
  MALOQ_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & al) == 0,
                "x and out must be %d-byte aligned", static_cast<int>(al + 1));
  rot::Args a{};
  a.x = x; a.gather = gather; a.E = num_edges; a.C = c; a.eulers = eulers; a.wigner = wigner;
  a.jd = jd; a.inverse = inverse; a.out = out;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (lmax) {
    case 0: return rot::launch<0>(x_dtype, out_dtype, a, s);
    case 1: return rot::launch<1>(x_dtype, out_dtype, a, s);
    case 2: return rot::launch<2>(x_dtype, out_dtype, a, s);
    case 3: return rot::launch<3>(x_dtype, out_dtype, a, s);
    case 4: return rot::launch<4>(x_dtype, out_dtype, a, s);
    case 5: return rot::launch<5>(x_dtype, out_dtype, a, s);
    case 6: return rot::launch<6>(x_dtype, out_dtype, a, s);
    case 7: return rot::launch<7>(x_dtype, out_dtype, a, s);
    default: return rot::launch<8>(x_dtype, out_dtype, a, s);
  }
}
