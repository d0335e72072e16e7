// Fused RadialMLP of the SO(2) convolution (gfx950).
//
// Reference: RadialMLP (radial.py:115-142), applied to the edge features at
// so2_layers.py:152-154 (its output scales the rotated rows, :160-163,191-198):
//   u_0 = x_edge;  u_i = SiLU(LayerNorm_i(W_i u_{i-1} + b_i)),  i = 1..H;
//   rad = W_o u_H + b_o.
// LayerNorm is torch's (biased variance, eps inside the square root, affine).
//
// Forward (radial_fwd_kernel): one workgroup of 4 waves per 64 edges, one edge
// per lane.  Hidden layers run on the VALU in fp32 from LDS rows (the weights
// are wave-uniform, so they arrive through scalar loads); the row statistics
// of LayerNorm are summed across the 4 waves in a fixed order.  The output
// layer is an MFMA GEMM in the dtype of the message rows (bf16 with fp32
// accumulation, or fp32): rad^T tile [32 outputs x 32 edges] =
// W_o[32 x c_H] u_H^T, the W_o fragments read straight from global memory in
// MFMA lane order, the u_H fragments built once from LDS.  Optionally saves
// u_H for the weight gradient.
//
// Backward: radial_bwd_kernel recomputes the hidden chain of its 64 edges,
// forms du_H = G W_o on the MFMA (G = dL/drad rows read once, the K range
// split over the 4 waves and summed in wave order), then runs the chain
// backward on the VALU (SiLU', LayerNorm backward, du_{i-1} = W_i^T dz_i) and
// writes per-workgroup partials of dW_i, db_i, dgamma_i, dbeta_i.
// radial_dwo_kernel forms dW_o = G^T u_H and db_o = G^T 1 split over edge
// ranges (bf16: natural [edge][channel] LDS tiles read back transposed with
// ds_read_b64_tr_b16; fp32: 32x32x2 MFMA operands loaded directly), and
// radial_reduce_kernel sums the partials in a fixed order.  Deterministic,
// no atomics.
#include "message_impl.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace rad {

using msg::BF16;
using msg::F32;
using msg::f32x16;
using msg::bf16x8;

typedef unsigned int frag_t __attribute__((ext_vector_type(4)));

constexpr int MAXH = 3;     // hidden layers
constexpr int TE = 64;      // edges per workgroup (one per lane)
constexpr int NT = 256;     // threads per workgroup
constexpr int MAXC = 128;   // widest input / hidden layer
constexpr int LDS_MAX = 160 * 1024;

struct Args {
  const float* x;  // [E, c0]
  int64_t E;
  int nh;
  int c[MAXH + 2];  // c0, c1 .. cH, c_out
  const float* w[MAXH];
  const float* b[MAXH];
  const float* g[MAXH];
  const float* bt[MAXH];
  float eps;
  const void* wo;   // [c_out, c_H] (TM raw)
  const void* wot;  // [c_H, c_out] (TM raw)
  const float* bo;  // [c_out]
  void* out;        // forward: [E, c_out] (TM raw)
  void* save;       // forward: [E, c_H] (TM raw), nullable
  const void* grad; // backward: [E, c_out] (TM raw)
  float* dx;        // backward: [E, c0], nullable
  float* part;      // backward partials
  int64_t pstride;  // floats per workgroup partial
  int64_t e_per_split;
};

__host__ __device__ constexpr int pitch(int c) { return c + 4; }  // LDS row pitch (floats)

__device__ __forceinline__ void mfma(f32x16& acc, frag_t a, frag_t b, BF16) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16((bf16x8)a, (bf16x8)b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mfma(f32x16& acc, frag_t a, frag_t b, F32) {
  // float j of lane half h is K index (j, h) in A and B alike
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

// VEC consecutive fp32 values -> one fragment of TM raw elements.
__device__ __forceinline__ frag_t pack_frag(const float* p, BF16) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  frag_t f;
  f.x = f32_to_bf16(a.x) | (static_cast<uint32_t>(f32_to_bf16(a.y)) << 16);
  f.y = f32_to_bf16(a.z) | (static_cast<uint32_t>(f32_to_bf16(a.w)) << 16);
  f.z = f32_to_bf16(b.x) | (static_cast<uint32_t>(f32_to_bf16(b.y)) << 16);
  f.w = f32_to_bf16(b.z) | (static_cast<uint32_t>(f32_to_bf16(b.w)) << 16);
  return f;
}
__device__ __forceinline__ frag_t pack_frag(const float* p, F32) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  frag_t f;
  f.x = __float_as_uint(a.x);
  f.y = __float_as_uint(a.y);
  f.z = __float_as_uint(a.z);
  f.w = __float_as_uint(a.w);
  return f;
}

__device__ __forceinline__ float silu(float a) { return a / (1.0f + expf(-a)); }

// ---------------------------------------------------------------- hidden chain
// Layer z = W ain + b for every edge of the tile (lane = edge) and the wave's
// quarter of the outputs, then LayerNorm over each row and SiLU.
// z and then xhat go to xh (pitch pitch(c)); rstd to rs (if non-null);
// u = SiLU(gamma xhat + beta) to aout (if non-null).
__device__ __forceinline__ void hidden_fwd(const float* __restrict__ W, const float* __restrict__ bias,
                                           const float* __restrict__ gam, const float* __restrict__ bet,
                                           int cin, int c, const float* ain, float* xh, float* rs,
                                           float* aout, float* red, float eps, int wave, int lane) {
  const int q = c >> 2, j0 = wave * q;
  const float* ar = ain + lane * pitch(cin);
  float* xr = xh + lane * pitch(c);
  float s1 = 0.f;
  for (int jc = 0; jc < q; jc += 4) {
    const int j = j0 + jc;
    float z0 = bias[j], z1 = bias[j + 1], z2 = bias[j + 2], z3 = bias[j + 3];
    const float* w0 = W + static_cast<int64_t>(j) * cin;
    for (int k = 0; k < cin; k += 4) {
      const float4 a4 = *reinterpret_cast<const float4*>(ar + k);
      const float4 u0 = *reinterpret_cast<const float4*>(w0 + k);
      const float4 u1 = *reinterpret_cast<const float4*>(w0 + cin + k);
      const float4 u2 = *reinterpret_cast<const float4*>(w0 + 2 * cin + k);
      const float4 u3 = *reinterpret_cast<const float4*>(w0 + 3 * cin + k);
      z0 = fmaf(u0.x, a4.x, z0); z0 = fmaf(u0.y, a4.y, z0); z0 = fmaf(u0.z, a4.z, z0); z0 = fmaf(u0.w, a4.w, z0);
      z1 = fmaf(u1.x, a4.x, z1); z1 = fmaf(u1.y, a4.y, z1); z1 = fmaf(u1.z, a4.z, z1); z1 = fmaf(u1.w, a4.w, z1);
      z2 = fmaf(u2.x, a4.x, z2); z2 = fmaf(u2.y, a4.y, z2); z2 = fmaf(u2.z, a4.z, z2); z2 = fmaf(u2.w, a4.w, z2);
      z3 = fmaf(u3.x, a4.x, z3); z3 = fmaf(u3.y, a4.y, z3); z3 = fmaf(u3.z, a4.z, z3); z3 = fmaf(u3.w, a4.w, z3);
    }
    *reinterpret_cast<float4*>(xr + j) = make_float4(z0, z1, z2, z3);
    s1 += (z0 + z1) + (z2 + z3);
  }
  red[wave * TE + lane] = s1;
  __syncthreads();
  const float inv_c = 1.0f / static_cast<float>(c);
  const float mean = ((red[lane] + red[TE + lane]) + (red[2 * TE + lane] + red[3 * TE + lane])) * inv_c;
  float s2 = 0.f;
  for (int jc = 0; jc < q; jc += 4) {
    const float4 z = *reinterpret_cast<const float4*>(xr + j0 + jc);
    const float d0 = z.x - mean, d1 = z.y - mean, d2 = z.z - mean, d3 = z.w - mean;
    s2 += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
  }
  red[4 * TE + wave * TE + lane] = s2;
  __syncthreads();
  const float var = ((red[4 * TE + lane] + red[5 * TE + lane]) + (red[6 * TE + lane] + red[7 * TE + lane])) * inv_c;
  const float rstd = 1.0f / sqrtf(var + eps);
  if (rs != nullptr && wave == 0) rs[lane] = rstd;
  for (int jc = 0; jc < q; jc += 4) {
    const int j = j0 + jc;
    float4 z = *reinterpret_cast<const float4*>(xr + j);
    z.x = (z.x - mean) * rstd; z.y = (z.y - mean) * rstd; z.z = (z.z - mean) * rstd; z.w = (z.w - mean) * rstd;
    *reinterpret_cast<float4*>(xr + j) = z;
    if (aout != nullptr) {
      float4 u;
      u.x = silu(fmaf(gam[j], z.x, bet[j]));
      u.y = silu(fmaf(gam[j + 1], z.y, bet[j + 1]));
      u.z = silu(fmaf(gam[j + 2], z.z, bet[j + 2]));
      u.w = silu(fmaf(gam[j + 3], z.w, bet[j + 3]));
      *reinterpret_cast<float4*>(aout + lane * pitch(c) + j) = u;
    }
  }
  __syncthreads();  // red reusable; rows complete for every wave
}

// Input rows of the tile (zero beyond the last edge).
__device__ __forceinline__ void load_input(const Args& a, float* act0, int64_t e0, int nvalid, int tid) {
  const int c0 = a.c[0], n4 = c0 >> 2;
  for (int i = tid; i < TE * n4; i += NT) {
    const int e = i / n4, k = (i - e * n4) * 4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (e < nvalid) v = *reinterpret_cast<const float4*>(a.x + (e0 + e) * c0 + k);
    *reinterpret_cast<float4*>(act0 + e * pitch(c0) + k) = v;
  }
  __syncthreads();
}

// ---------------------------------------------------------------- forward
template <class TM>
__global__ __launch_bounds__(NT) void radial_fwd_kernel(Args a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  using raw = typename TM::raw;
  constexpr int KC = TM::KC, VEC = TM::VEC;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * TE;
  const int nvalid = static_cast<int>((a.E - e0) < TE ? (a.E - e0) : TE);
  int cmax = 0;
  for (int i = 1; i <= a.nh; ++i) cmax = a.c[i] > cmax ? a.c[i] : cmax;
  float* red = smem;                          // [8][TE]
  float* act0 = red + 8 * TE;                 // [TE][pitch(c0)]
  float* buf0 = act0 + TE * pitch(a.c[0]);    // [TE][pitch(cmax)] x2: xhat / activations
  float* buf1 = buf0 + TE * pitch(cmax);
  load_input(a, act0, e0, nvalid, tid);
  const float* ain = act0;
  float* cur = buf0;
  float* other = buf1;
  for (int i = 0; i < a.nh; ++i) {
    // z / xhat and u share the buffer: each lane's row is normalised and
    // activated in place after its statistics are known
    hidden_fwd(a.w[i], a.b[i], a.g[i], a.bt[i], a.c[i], a.c[i + 1], ain, cur, nullptr, cur, red,
               a.eps, wave, lane);
    ain = cur;
    float* t = cur;
    cur = other;
    other = t;
  }
  const int cH = a.c[a.nh], cout = a.c[a.nh + 1];
  const float* uH = ain;  // [TE][pitch(cH)]
  // saved u_H rows (TM raw) for the weight gradient
  if (a.save != nullptr && lane < nvalid) {
    raw* sv = reinterpret_cast<raw*>(a.save) + (e0 + lane) * cH;
    const int q = cH >> 2;
    for (int j = wave * q; j < (wave + 1) * q; j += VEC) {
      const frag_t f = pack_frag(uH + lane * pitch(cH) + j, TM{});
      *reinterpret_cast<frag_t*>(sv + j) = f;
    }
  }
  // B fragments: u_H^T, lane (edge 32 nt + lane % 32, K half lane / 32)
  constexpr int NKMAX = MAXC / KC;
  const int nk = cH / KC;
  frag_t bf[2][NKMAX];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int kc = 0; kc < NKMAX; ++kc)
      if (kc < nk) bf[nt][kc] = pack_frag(uH + (32 * nt + (lane & 31)) * pitch(cH) + kc * KC + (lane >> 5) * VEC, TM{});
  const raw* wo = reinterpret_cast<const raw*>(a.wo);
  raw* out = reinterpret_cast<raw*>(a.out);
  const int not_ = cout / 32;
  for (int ot = wave; ot < not_; ot += 4) {
    const int o0 = ot * 32;
    frag_t af[NKMAX];
    const raw* wrow = wo + static_cast<int64_t>(o0 + (lane & 31)) * cH + (lane >> 5) * VEC;
#pragma unroll
    for (int kc = 0; kc < NKMAX; ++kc)
      if (kc < nk) af[kc] = *reinterpret_cast<const frag_t*>(wrow + kc * KC);
    f32x16 acc[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[nt][r] = 0.f;
#pragma unroll
    for (int kc = 0; kc < NKMAX; ++kc)
      if (kc < nk) {
        mfma(acc[0], af[kc], bf[0][kc], TM{});
        mfma(acc[1], af[kc], bf[1][kc], TM{});
      }
    // lane L, register r: output o0 + 8 (r/4) + 4 (L/32) + r%4, edge 32 nt + L%32
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int e = 32 * nt + (lane & 31);
      if (e < nvalid) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int o = o0 + 8 * g4 + 4 * (lane >> 5);
          const float4 bb = *reinterpret_cast<const float4*>(a.bo + o);
          raw* dst = out + (e0 + e) * cout + o;
          const float v0 = acc[nt][4 * g4] + bb.x, v1 = acc[nt][4 * g4 + 1] + bb.y;
          const float v2 = acc[nt][4 * g4 + 2] + bb.z, v3 = acc[nt][4 * g4 + 3] + bb.w;
          if constexpr (sizeof(raw) == 2) {
            uint2 w;
            w.x = f32_to_bf16(v0) | (static_cast<uint32_t>(f32_to_bf16(v1)) << 16);
            w.y = f32_to_bf16(v2) | (static_cast<uint32_t>(f32_to_bf16(v3)) << 16);
            *reinterpret_cast<uint2*>(dst) = w;
          } else {
            *reinterpret_cast<float4*>(dst) = make_float4(v0, v1, v2, v3);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------- backward (tile)
template <class TM>
__global__ __launch_bounds__(NT) void radial_bwd_kernel(Args a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  using raw = typename TM::raw;
  constexpr int KC = TM::KC, VEC = TM::VEC;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * TE;
  const int nvalid = static_cast<int>((a.E - e0) < TE ? (a.E - e0) : TE);
  const int nh = a.nh, cH = a.c[nh], cout = a.c[nh + 1];
  int cmax = a.c[0];
  for (int i = 1; i <= nh; ++i) cmax = a.c[i] > cmax ? a.c[i] : cmax;
  float* red = smem;                        // [8][TE]
  float* rs = red + 8 * TE;                 // [MAXH][TE] rstd per layer
  float* act0 = rs + MAXH * TE;             // [TE][pitch(c0)]
  float* xh[MAXH];                          // [TE][pitch(c_i)] xhat per layer
  float* p = act0 + TE * pitch(a.c[0]);
  for (int i = 0; i < nh; ++i) {
    xh[i] = p;
    p += TE * pitch(a.c[i + 1]);
  }
  float* du = p;                            // [TE][pitch(cmax)]
  float* dz = du + TE * pitch(cmax);
  float* at = dz + TE * pitch(cmax);        // recomputed activations
  load_input(a, act0, e0, nvalid, tid);

  // recompute the chain: xhat and rstd of every layer
  {
    const float* ain = act0;
    for (int i = 0; i < nh; ++i) {
      float* aout = (i + 1 < nh) ? ((i & 1) ? du : at) : nullptr;
      hidden_fwd(a.w[i], a.b[i], a.g[i], a.bt[i], a.c[i], a.c[i + 1], ain, xh[i], rs + i * TE, aout,
                 red, a.eps, wave, lane);
      ain = aout;
    }
  }

  // du_H [e][j] = sum_o G[e][o] W_o[o][j]: waves split the K (output) range
  {
    const raw* G = reinterpret_cast<const raw*>(a.grad);
    const raw* wot = reinterpret_cast<const raw*>(a.wot);
    const int nks = cout / KC, kq = nks / 4, ks0 = wave * kq;
    const int nnt = cH / 32;
    constexpr int NNT = MAXC / 32;
    f32x16 acc[2][NNT];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.f;
    const raw* ga[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      int e = 32 * mt + (lane & 31);
      e = e < nvalid ? e : nvalid - 1;  // in-bounds rows; results of padded edges are never used
      ga[mt] = G + (e0 + e) * cout + (lane >> 5) * VEC;
    }
    const raw* gb = wot + static_cast<int64_t>(lane & 31) * cout + (lane >> 5) * VEC;
    for (int ks = ks0; ks < ks0 + kq; ++ks) {
      frag_t fa[2], fb[NNT];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) fa[mt] = *reinterpret_cast<const frag_t*>(ga[mt] + ks * KC);
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
        if (nt < nnt) fb[nt] = *reinterpret_cast<const frag_t*>(gb + static_cast<int64_t>(32 * nt) * cout + ks * KC);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < NNT; ++nt)
          if (nt < nnt) mfma(acc[mt][nt], fa[mt], fb[nt], TM{});
    }
    // sum over waves in wave order: lane L, register r -> edge 32 mt + 8 (r/4) + 4 (L/32) + r%4,
    // column 32 nt + L%32
    for (int w = 0; w < 4; ++w) {
      if (wave == w) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int nt = 0; nt < NNT; ++nt)
            if (nt < nnt)
#pragma unroll
              for (int r = 0; r < 16; ++r) {
                const int e = 32 * mt + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float* d = du + e * pitch(cH) + 32 * nt + (lane & 31);
                *d = (w == 0) ? acc[mt][nt][r] : *d + acc[mt][nt][r];
              }
      }
      __syncthreads();
    }
  }

  // chain backward
  float* part = a.part + static_cast<int64_t>(blockIdx.x) * a.pstride;
  int64_t poff = 0;
  for (int i = 0; i < nh; ++i) poff += static_cast<int64_t>(a.c[i + 1]) * (a.c[i] + 3);
  const bool valid = lane < nvalid;
  for (int i = nh - 1; i >= 0; --i) {
    const int c = a.c[i + 1], cin = a.c[i], q = c >> 2, j0 = wave * q;
    const float* gam = a.g[i];
    const float* bet = a.bt[i];
    const float* xr = xh[i] + lane * pitch(c);
    float* dur = du + lane * pitch(c);
    float* dzr = dz + lane * pitch(c);
    // da = du * SiLU'(a); dah = da * gamma -> du (da) and dz (dah) rows
    float s1 = 0.f, s2 = 0.f;
    for (int jc = 0; jc < q; jc += 4) {
      const int j = j0 + jc;
      const float4 x4 = *reinterpret_cast<const float4*>(xr + j);
      const float4 d4 = *reinterpret_cast<const float4*>(dur + j);
      float xv[4] = {x4.x, x4.y, x4.z, x4.w}, dv[4] = {d4.x, d4.y, d4.z, d4.w}, da[4], dh[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float av = fmaf(gam[j + t], xv[t], bet[j + t]);
        const float sg = 1.0f / (1.0f + expf(-av));
        da[t] = valid ? dv[t] * (sg * (1.0f + av * (1.0f - sg))) : 0.f;
        dh[t] = da[t] * gam[j + t];
        s1 += dh[t];
        s2 += dh[t] * xv[t];
      }
      *reinterpret_cast<float4*>(dur + j) = make_float4(da[0], da[1], da[2], da[3]);
      *reinterpret_cast<float4*>(dzr + j) = make_float4(dh[0], dh[1], dh[2], dh[3]);
    }
    red[wave * TE + lane] = s1;
    red[4 * TE + wave * TE + lane] = s2;
    __syncthreads();
    const float inv_c = 1.0f / static_cast<float>(c);
    const float m1 = ((red[lane] + red[TE + lane]) + (red[2 * TE + lane] + red[3 * TE + lane])) * inv_c;
    const float m2 = ((red[4 * TE + lane] + red[5 * TE + lane]) + (red[6 * TE + lane] + red[7 * TE + lane])) * inv_c;
    const float rstd = rs[i * TE + lane];
    for (int jc = 0; jc < q; jc += 4) {
      const int j = j0 + jc;
      const float4 x4 = *reinterpret_cast<const float4*>(xr + j);
      float4 h = *reinterpret_cast<const float4*>(dzr + j);
      h.x = rstd * (h.x - m1 - x4.x * m2);
      h.y = rstd * (h.y - m1 - x4.y * m2);
      h.z = rstd * (h.z - m1 - x4.z * m2);
      h.w = rstd * (h.w - m1 - x4.w * m2);
      *reinterpret_cast<float4*>(dzr + j) = h;
    }
    // activations feeding layer i (u_{i}) for its weight gradient
    if (i > 0) {
      const int cp = a.c[i], qp = cp >> 2, jp = wave * qp;
      const float* gp = a.g[i - 1];
      const float* bp = a.bt[i - 1];
      const float* xp = xh[i - 1] + lane * pitch(cp);
      for (int j = jp; j < jp + qp; ++j) at[lane * pitch(cp) + j] = silu(fmaf(gp[j], xp[j], bp[j]));
    }
    __syncthreads();
    const float* ain = (i > 0) ? at : act0;
    poff -= static_cast<int64_t>(c) * (cin + 3);
    float* pw = part + poff;  // dW_i [c][cin], then db_i, dgamma_i, dbeta_i
    // column sums over the tile's edges (fixed order)
    for (int j = tid; j < c; j += NT) {
      float sb = 0.f, sgm = 0.f, sbt = 0.f;
      for (int e = 0; e < TE; ++e) {
        const float dav = du[e * pitch(c) + j];
        sb += dz[e * pitch(c) + j];
        sbt += dav;
        sgm += dav * xh[i][e * pitch(c) + j];
      }
      pw[c * cin + j] = sb;
      pw[c * cin + c + j] = sgm;
      pw[c * cin + 2 * c + j] = sbt;
    }
    // dW_i [j][k] = sum_e dz[e][j] u[e][k], 4 x 4 blocks per thread
    {
      const int nbj = c >> 2, nbk = cin >> 2;
      for (int blk = tid; blk < nbj * nbk; blk += NT) {
        const int jb = (blk / nbk) * 4, kb = (blk % nbk) * 4;
        float acc[4][4] = {};
        for (int e = 0; e < TE; ++e) {
          const float4 z4 = *reinterpret_cast<const float4*>(dz + e * pitch(c) + jb);
          const float4 u4 = *reinterpret_cast<const float4*>(ain + e * pitch(cin) + kb);
          const float zv[4] = {z4.x, z4.y, z4.z, z4.w}, uv[4] = {u4.x, u4.y, u4.z, u4.w};
#pragma unroll
          for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int t = 0; t < 4; ++t) acc[s][t] = fmaf(zv[s], uv[t], acc[s][t]);
        }
#pragma unroll
        for (int s = 0; s < 4; ++s)
          *reinterpret_cast<float4*>(pw + (jb + s) * cin + kb) = make_float4(acc[s][0], acc[s][1], acc[s][2], acc[s][3]);
      }
    }
    __syncthreads();  // du / at free again
    // du_{i-1} [e][k] = sum_j dz[e][j] W_i[j][k]  (into du, or dx for the input)
    if (i > 0 || a.dx != nullptr) {
      const float* W = a.w[i];
      for (int ch = wave; ch < (cin >> 2); ch += 4) {  // 4-column chunks, round-robin over waves
        const int k = 4 * ch;
        float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int j = 0; j < c; ++j) {
          const float zj = dzr[j];
          const float4 w4 = *reinterpret_cast<const float4*>(W + static_cast<int64_t>(j) * cin + k);
          s.x = fmaf(zj, w4.x, s.x); s.y = fmaf(zj, w4.y, s.y); s.z = fmaf(zj, w4.z, s.z); s.w = fmaf(zj, w4.w, s.w);
        }
        if (i > 0)
          *reinterpret_cast<float4*>(du + lane * pitch(cin) + k) = s;
        else if (valid)
          *reinterpret_cast<float4*>(a.dx + (e0 + lane) * cin + k) = s;
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------- dW_o, db_o
// bf16: per 32-edge step, G [32 x 128 outputs] and u_H [32 x c_H] are staged
// in natural layout (row pitch padded by 64 bytes) and read back as MFMA
// operands of 8 consecutive edges per lane with ds_read_b64_tr_b16.
typedef short v4s16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s16 lds_v4s16;

__device__ __forceinline__ v4s16 tr_read(const char* lds) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4s16*)((__attribute__((address_space(3))) const char*)lds));
}

constexpr int DO_T = 128;   // outputs per workgroup tile
constexpr int DO_KE = 32;   // edges per step

template <class TM>
__global__ __launch_bounds__(NT) void radial_dwo_kernel(Args a);

template <>
__global__ __launch_bounds__(NT) void radial_dwo_kernel<BF16>(Args a) {
  constexpr int PG = DO_T * 2 + 64;  // bytes per staged G row
  constexpr int PU = MAXC * 2 + 64;  // bytes per staged u row (upper bound)
  __shared__ alignas(16) char sg[2][DO_KE * PG];
  __shared__ alignas(16) char su[2][DO_KE * PU];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nh = a.nh, cH = a.c[nh], cout = a.c[nh + 1];
  const int not_ = (cout + DO_T - 1) / DO_T;
  const int ot = blockIdx.x % not_;
  const int64_t split = blockIdx.x / not_;
  const int o0 = ot * DO_T;
  const int64_t eb = split * a.e_per_split;
  const int64_t ee = (eb + a.e_per_split) < a.E ? (eb + a.e_per_split) : a.E;
  const int nsteps = ee > eb ? static_cast<int>((ee - eb + DO_KE - 1) / DO_KE) : 0;
  const int pu = cH * 2 + 64;
  const uint16_t* G = reinterpret_cast<const uint16_t*>(a.grad);
  const uint16_t* U = reinterpret_cast<const uint16_t*>(a.save);
  // loads: G chunk (row, 16-byte column) = tid + 256 t (t = 0, 1); u chunk tid + 256 t (< 32 cH/8)
  const int ucols = cH / 8;
  uint4 rg[2], ru[2];
  auto load = [&](int step) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ch = tid + NT * t, r = ch >> 4, col = (ch & 15) * 8;
      const int64_t e = eb + static_cast<int64_t>(step) * DO_KE + r;
      rg[t] = make_uint4(0u, 0u, 0u, 0u);
      if (e < ee && o0 + col < cout) rg[t] = *reinterpret_cast<const uint4*>(G + e * cout + o0 + col);
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ch = tid + NT * t;
      ru[t] = make_uint4(0u, 0u, 0u, 0u);
      if (ch < DO_KE * ucols) {
        const int r = ch / ucols, col = (ch % ucols) * 8;
        const int64_t e = eb + static_cast<int64_t>(step) * DO_KE + r;
        if (e < ee) ru[t] = *reinterpret_cast<const uint4*>(U + e * cH + col);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ch = tid + NT * t, r = ch >> 4, col = ch & 15;
      *reinterpret_cast<uint4*>(sg[buf] + r * PG + col * 16) = rg[t];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int ch = tid + NT * t;
      if (ch < DO_KE * ucols) {
        const int r = ch / ucols, col = ch % ucols;
        *reinterpret_cast<uint4*>(su[buf] + r * pu + col * 16) = ru[t];
      }
    }
  };
  constexpr int NNT = MAXC / 32;
  const int nnt = cH / 32;
  f32x16 acc[NNT], accb;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    accb[r] = 0.f;
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt) acc[nt][r] = 0.f;
  }
  const bf16x8 ones = {0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x3F80};
  // transposed reads: lane (g16, a, kk) addresses row 8 (g16/2) + 4 r + kk, column 16 (g16%2) + 4 a
  const int g16 = lane >> 4, aa = lane & 3, kk = (lane >> 2) & 3;
  const int rowl = 8 * (g16 >> 1) + kk, coll = 16 * (g16 & 1) + 4 * aa;
  const bool active = o0 + 32 * wave < cout;
  if (nsteps > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int s = 0; s < nsteps; ++s) {
    const int cb = s & 1;
    if (s + 1 < nsteps) load(s + 1);
    if (active) {
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const char* ga = sg[cb] + (16 * sub + rowl) * PG + (32 * wave + coll) * 2;
        const v4s16 a0 = tr_read(ga), a1 = tr_read(ga + 4 * PG);
        const bf16x8 af = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
        accb = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, ones, accb, 0, 0, 0);
#pragma unroll
        for (int nt = 0; nt < NNT; ++nt)
          if (nt < nnt) {
            const char* ub = su[cb] + (16 * sub + rowl) * pu + (32 * nt + coll) * 2;
            const v4s16 b0 = tr_read(ub), b1 = tr_read(ub + 4 * pu);
            const bf16x8 bfv = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
            acc[nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bfv, acc[nt], 0, 0, 0);
          }
      }
    }
    if (s + 1 < nsteps) store(cb ^ 1);
    __syncthreads();
  }
  if (!active) return;
  float* part = a.part + split * a.pstride;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int o = o0 + 32 * wave + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
      if (nt < nnt) part[static_cast<int64_t>(o) * cH + 32 * nt + (lane & 31)] = acc[nt][r];
    if ((lane & 31) == 0) part[static_cast<int64_t>(cout) * cH + o] = accb[r];
  }
}

template <>
__global__ __launch_bounds__(NT) void radial_dwo_kernel<F32>(Args a) {
  // 32x32x2 fp32 MFMA: lane i supplies A[o = i%32][edge i/32] and B[edge i/32][j = i%32],
  // both straight from the natural rows
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nh = a.nh, cH = a.c[nh], cout = a.c[nh + 1];
  const int not_ = (cout + DO_T - 1) / DO_T;
  const int ot = blockIdx.x % not_;
  const int64_t split = blockIdx.x / not_;
  const int o = ot * DO_T + 32 * wave + (lane & 31);
  if (ot * DO_T + 32 * wave >= cout) return;
  const int64_t eb = split * a.e_per_split;
  const int64_t ee = (eb + a.e_per_split) < a.E ? (eb + a.e_per_split) : a.E;
  const float* G = reinterpret_cast<const float*>(a.grad);
  const float* U = reinterpret_cast<const float*>(a.save);
  constexpr int NNT = MAXC / 32;
  const int nnt = cH / 32;
  f32x16 acc[NNT], accb;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    accb[r] = 0.f;
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt) acc[nt][r] = 0.f;
  }
  const int h = lane >> 5;
  for (int64_t e = eb; e < ee; e += 2) {
    const int64_t er = e + h;
    const bool ok = er < ee;
    const float av = ok ? G[er * cout + o] : 0.f;
    accb = __builtin_amdgcn_mfma_f32_32x32x2f32(av, 1.0f, accb, 0, 0, 0);
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
      if (nt < nnt) {
        const float bv = ok ? U[er * cH + 32 * nt + (lane & 31)] : 0.f;
        acc[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc[nt], 0, 0, 0);
      }
  }
  float* part = a.part + split * a.pstride;
  const int ob = ot * DO_T + 32 * wave;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int oo = ob + 8 * (r >> 2) + 4 * h + (r & 3);
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
      if (nt < nnt) part[static_cast<int64_t>(oo) * cH + 32 * nt + (lane & 31)] = acc[nt][r];
    if ((lane & 31) == 0) part[static_cast<int64_t>(cout) * cH + oo] = accb[r];
  }
}

// out[k] = sum over n partial vectors (stride floats apart), in order; 8
// interleaved running sums combined in a fixed order.
__global__ void radial_reduce_kernel(const float* __restrict__ part, int64_t n, int64_t nparts,
                                     int64_t stride, float* __restrict__ out0, int64_t n0,
                                     float* __restrict__ out1) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k >= n) return;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t p = 0;
  for (; p + 8 <= nparts; p += 8)
#pragma unroll
    for (int t = 0; t < 8; ++t) s[t] += part[(p + t) * stride + k];
  for (int t = 0; p < nparts; ++p, ++t) s[t] += part[p * stride + k];
  const float v = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
  if (k < n0)
    out0[k] = v;
  else
    out1[k - n0] = v;
}

// W_o (fp32 [c_out, c_H]) -> wo (TM raw, same layout) and wot (TM raw [c_H, c_out]).
template <class TM>
__global__ void radial_pack_kernel(const float* __restrict__ w, int cout, int cH, void* wo, void* wot) {
  using raw = typename TM::raw;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(cout) * cH) return;
  const int o = static_cast<int>(i / cH), j = static_cast<int>(i % cH);
  const raw v = TM::cvt(w[i]);
  if (wo != nullptr) reinterpret_cast<raw*>(wo)[i] = v;
  reinterpret_cast<raw*>(wot)[static_cast<int64_t>(j) * cout + o] = v;
}

}  // namespace rad
}  // namespace maloq

using namespace maloq;
using namespace maloq::rad;

static int64_t fwd_lds(const Args& a) {
  int cmax = 0;
  for (int i = 1; i <= a.nh; ++i) cmax = a.c[i] > cmax ? a.c[i] : cmax;
  return 4 * (8 * TE + static_cast<int64_t>(TE) * (pitch(a.c[0]) + 2 * pitch(cmax)));
}
static int64_t bwd_lds(const Args& a) {
  int cmax = a.c[0];
  for (int i = 1; i <= a.nh; ++i) cmax = a.c[i] > cmax ? a.c[i] : cmax;
  int64_t f = 8 * TE + MAXH * TE + static_cast<int64_t>(TE) * pitch(a.c[0]);
  for (int i = 1; i <= a.nh; ++i) f += static_cast<int64_t>(TE) * pitch(a.c[i]);
  f += 3 * static_cast<int64_t>(TE) * pitch(cmax);
  return 4 * f;
}
static int64_t hidden_grad_floats(const Args& a) {
  int64_t s = 0;
  for (int i = 0; i < a.nh; ++i) s += static_cast<int64_t>(a.c[i + 1]) * (a.c[i] + 3);
  return s;
}
static int dwo_splits(const Args& a) {
  const int not_ = (a.c[a.nh + 1] + DO_T - 1) / DO_T;
  int s = 512 / not_;
  const int64_t smax = (a.E + 255) / 256;  // at least 256 edges per split
  if (s > smax) s = static_cast<int>(smax);
  return s < 1 ? 1 : (s > 128 ? 128 : s);
}

// Dynamic LDS above the default limit needs the kernel's attribute raised first.
static int dyn_lds(const void* fn, size_t bytes) {
  if (bytes <= 64 * 1024) return MALOQ_OK;
  const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
  MALOQ_REQUIRE(e == hipSuccess, "hipFuncSetAttribute(max dynamic LDS %zu): %s", bytes, hipGetErrorString(e));
  return MALOQ_OK;
}

static int setup(Args& a, int dtype, int nhidden, const int* widths, int64_t E) {
  MALOQ_REQUIRE(dtype == 0 || dtype == 1, "dtype must be 0 (fp32) or 1 (bf16)");
  MALOQ_REQUIRE(nhidden >= 1 && nhidden <= MAXH, "RadialMLP: 1..%d hidden layers supported", MAXH);
  MALOQ_REQUIRE(widths != nullptr, "widths is null");
  MALOQ_REQUIRE(E >= 0, "num_edges < 0");
  a = Args{};
  a.E = E;
  a.nh = nhidden;
  for (int i = 0; i < nhidden + 2; ++i) a.c[i] = widths[i];
  MALOQ_REQUIRE(a.c[0] >= 4 && a.c[0] % 4 == 0 && a.c[0] <= MAXC,
                "RadialMLP input width %d: a multiple of 4 up to %d is supported", a.c[0], MAXC);
  for (int i = 1; i <= nhidden; ++i)
    MALOQ_REQUIRE(a.c[i] >= 32 && a.c[i] % 32 == 0 && a.c[i] <= MAXC,
                  "RadialMLP hidden width %d: a multiple of 32 up to %d is supported", a.c[i], MAXC);
  MALOQ_REQUIRE(a.c[nhidden + 1] >= 64 && a.c[nhidden + 1] % 64 == 0,
                "RadialMLP output width %d must be a multiple of 64", a.c[nhidden + 1]);
  MALOQ_REQUIRE(bwd_lds(a) <= LDS_MAX, "RadialMLP widths need %lld bytes of LDS per workgroup (max %d)",
                static_cast<long long>(bwd_lds(a)), LDS_MAX);
  return MALOQ_OK;
}

static int set_params(Args& a, const float* const* w, const float* const* b, const float* const* g,
                      const float* const* bt, float eps) {
  MALOQ_REQUIRE(w && b && g && bt, "null parameter array");
  for (int i = 0; i < a.nh; ++i) {
    MALOQ_REQUIRE(w[i] && b[i] && g[i] && bt[i], "null parameter of hidden layer %d", i);
    MALOQ_REQUIRE((reinterpret_cast<uintptr_t>(w[i]) & 15) == 0, "hidden weight %d must be 16-byte aligned", i);
    a.w[i] = w[i];
    a.b[i] = b[i];
    a.g[i] = g[i];
    a.bt[i] = bt[i];
  }
  MALOQ_REQUIRE(eps > 0.f, "eps must be positive");
  a.eps = eps;
  return MALOQ_OK;
}

extern "C" int64_t maloq_radial_pack_bytes(int dtype, int c_out, int c_hidden) {
  if (dtype != 0 && dtype != 1) return -1;
  return 2 * static_cast<int64_t>(c_out) * c_hidden * (dtype == 1 ? 2 : 4);
}

extern "C" int64_t maloq_radial_bwd_partials_floats(int dtype, int nhidden, const int* widths,
                                                    int64_t num_edges) {
  Args a;
  if (setup(a, dtype, nhidden, widths, num_edges)) return -1;
  const int64_t ntiles = (num_edges + TE - 1) / TE;
  const int cH = a.c[a.nh], cout = a.c[a.nh + 1];
  const int64_t h = ntiles * hidden_grad_floats(a);
  const int64_t o = static_cast<int64_t>(dwo_splits(a)) * (static_cast<int64_t>(cout) * cH + cout);
  return (h > o ? h : o) + 1;
}

extern "C" int maloq_radial_fwd(int dtype, int nhidden, const int* widths, const float* x,
                                int64_t num_edges, const float* const* weight,
                                const float* const* bias, const float* const* ln_weight,
                                const float* const* ln_bias, float eps, const float* out_weight,
                                const float* out_bias, void* wpack, void* out, void* save,
                                void* stream) {
  Args a;
  int rc = setup(a, dtype, nhidden, widths, num_edges);
  if (rc) return rc;
  rc = set_params(a, weight, bias, ln_weight, ln_bias, eps);
  if (rc) return rc;
  MALOQ_REQUIRE(out_weight && out_bias && wpack, "null pointer");
  MALOQ_REQUIRE((reinterpret_cast<uintptr_t>(wpack) & 15) == 0 && (reinterpret_cast<uintptr_t>(out_bias) & 15) == 0,
                "wpack / out_bias must be 16-byte aligned");
  const int cH = a.c[a.nh], cout = a.c[a.nh + 1];
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t el = dtype == 1 ? 2 : 4;
  char* wo = static_cast<char*>(wpack);
  char* wot = wo + static_cast<size_t>(cout) * cH * el;
  const int64_t nw = static_cast<int64_t>(cout) * cH;
  // both layouts: the backward reads the transposed one from the same buffer
  if (dtype == 1)
    hipLaunchKernelGGL(radial_pack_kernel<BF16>, dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, s,
                       out_weight, cout, cH, static_cast<void*>(wo), static_cast<void*>(wot));
  else
    hipLaunchKernelGGL(radial_pack_kernel<F32>, dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, s,
                       out_weight, cout, cH, static_cast<void*>(wo), static_cast<void*>(wot));
  rc = check_launch("radial_pack_kernel");
  if (rc) return rc;
  if (num_edges == 0) return MALOQ_OK;
  MALOQ_REQUIRE(x && out, "null pointer");
  a.x = x;
  a.wo = wo;
  a.wot = wot;
  a.bo = out_bias;
  a.out = out;
  a.save = save;
  const int64_t ntiles = (num_edges + TE - 1) / TE;
  MALOQ_REQUIRE(ntiles < (int64_t(1) << 31), "too many edges");
  const size_t lds = static_cast<size_t>(fwd_lds(a));
  rc = dyn_lds(dtype == 1 ? reinterpret_cast<const void*>(&radial_fwd_kernel<BF16>)
                          : reinterpret_cast<const void*>(&radial_fwd_kernel<F32>), lds);
  if (rc) return rc;
  if (dtype == 1)
    hipLaunchKernelGGL(radial_fwd_kernel<BF16>, dim3(static_cast<unsigned>(ntiles)), dim3(NT), lds, s, a);
  else
    hipLaunchKernelGGL(radial_fwd_kernel<F32>, dim3(static_cast<unsigned>(ntiles)), dim3(NT), lds, s, a);
  return check_launch("radial_fwd_kernel");
}

extern "C" int maloq_radial_bwd(int dtype, int nhidden, const int* widths, const float* x,
                                int64_t num_edges, const float* const* weight,
                                const float* const* bias, const float* const* ln_weight,
                                const float* const* ln_bias, float eps, const void* wpack,
                                const void* grad, const void* save, float* grad_x,
                                float* partials, float* grad_hidden, float* grad_out_weight,
                                float* grad_out_bias, void* stream) {
  Args a;
  int rc = setup(a, dtype, nhidden, widths, num_edges);
  if (rc) return rc;
  rc = set_params(a, weight, bias, ln_weight, ln_bias, eps);
  if (rc) return rc;
  MALOQ_REQUIRE(wpack && partials && grad_hidden && grad_out_weight && grad_out_bias, "null pointer");
  MALOQ_REQUIRE(num_edges > 0, "the backward needs at least one edge (zero gradients otherwise)");
  MALOQ_REQUIRE(x && grad && save, "null pointer");
  const int cH = a.c[a.nh], cout = a.c[a.nh + 1];
  const size_t el = dtype == 1 ? 2 : 4;
  a.x = x;
  a.wo = wpack;
  a.wot = static_cast<const char*>(wpack) + static_cast<size_t>(cout) * cH * el;
  a.grad = grad;
  a.save = const_cast<void*>(save);  // read-only in the backward
  a.dx = grad_x;
  a.part = partials;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t ntiles = (num_edges + TE - 1) / TE;
  MALOQ_REQUIRE(ntiles < (int64_t(1) << 31), "too many edges");
  // hidden layers: per-tile partials, then their sum
  a.pstride = hidden_grad_floats(a);
  const size_t lds = static_cast<size_t>(bwd_lds(a));
  rc = dyn_lds(dtype == 1 ? reinterpret_cast<const void*>(&radial_bwd_kernel<BF16>)
                          : reinterpret_cast<const void*>(&radial_bwd_kernel<F32>), lds);
  if (rc) return rc;
  if (dtype == 1)
    hipLaunchKernelGGL(radial_bwd_kernel<BF16>, dim3(static_cast<unsigned>(ntiles)), dim3(NT), lds, s, a);
  else
    hipLaunchKernelGGL(radial_bwd_kernel<F32>, dim3(static_cast<unsigned>(ntiles)), dim3(NT), lds, s, a);
  rc = check_launch("radial_bwd_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(radial_reduce_kernel, dim3(static_cast<unsigned>((a.pstride + 255) / 256)), dim3(256), 0, s,
                     static_cast<const float*>(partials), a.pstride, ntiles, a.pstride, grad_hidden, a.pstride,
                     grad_hidden);
  rc = check_launch("radial_reduce_kernel");
  if (rc) return rc;
  // output layer: split-K partials of [dW_o | db_o], then their sum.  The
  // partials buffer is reused: stream order puts this after the reduce above.
  const int splits = dwo_splits(a);
  a.e_per_split = ((num_edges + splits - 1) / splits + DO_KE - 1) / DO_KE * DO_KE;
  a.pstride = static_cast<int64_t>(cout) * cH + cout;
  const int not_ = (cout + DO_T - 1) / DO_T;
  if (dtype == 1)
    hipLaunchKernelGGL(radial_dwo_kernel<BF16>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a);
  else
    hipLaunchKernelGGL(radial_dwo_kernel<F32>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a);
  rc = check_launch("radial_dwo_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(radial_reduce_kernel, dim3(static_cast<unsigned>((a.pstride + 255) / 256)), dim3(256), 0, s,
                     static_cast<const float*>(partials), a.pstride, static_cast<int64_t>(splits), a.pstride,
                     grad_out_weight, static_cast<int64_t>(cout) * cH, grad_out_bias);
  return check_launch("radial_reduce_kernel");
}
