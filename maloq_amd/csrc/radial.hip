// Fused RadialMLP of the SO(2) convolution (gfx950).
//
// Reference: RadialMLP (radial.py:115-142), applied to the edge features at
// so2_layers.py:152-154 (its output scales the rotated rows, :160-163,191-198):
//   u_0 = x_edge;  u_i = SiLU(LayerNorm_i(W_i u_{i-1} + b_i)),  i = 1..H;
//   rad = W_o u_H + b_o.
// LayerNorm is torch's (biased variance, eps inside the square root, affine).
//
// Forward (radial_fwd_kernel): one workgroup of 4 waves per 64 edges, one edge
// per lane.  The hidden layers' parameters are staged in LDS (weights
// transposed, so that a wave's block of outputs at one input is a broadcast
// 16-byte read); each lane keeps its quarter of the layer's outputs in
// registers, and the LayerNorm row statistics are summed across the 4 waves
// in a fixed order.  The output layer is an MFMA GEMM in the dtype of the
// message rows (bf16 with fp32 accumulation, or fp32): rad^T tile
// [32 outputs x 32 edges] = W_o[32 x c_H] u_H^T, W_o fragments read from
// global memory in MFMA lane order one tile ahead, u_H fragments built once
// from LDS.  Optionally saves u_H for the weight gradient.
//
// Backward:
//   radial_du_kernel     du_H = G W_o on the MFMA (G = dL/drad rows, read
//                        once; 64 edges per workgroup, the K range split over
//                        8 waves, partial tiles summed by a fixed tree).
//   radial_chain_kernel  recomputes the hidden chain of its 64 edges and runs
//                        it backward on the VALU (SiLU', LayerNorm backward,
//                        du_{i-1} = W_i^T dz_i), writing per-tile partials of
//                        dW_i, db_i, dgamma_i, dbeta_i (and dL/dx).
//   radial_dwo_kernel    dW_o = G^T u_H and db_o = G^T 1, split over edge
//                        ranges (bf16: natural [edge][channel] LDS tiles read
//                        back transposed with ds_read_b64_tr_b16; fp32: 32x32x2
//                        MFMA operands loaded directly).
//   radial_reduce*       sums of the partials in a fixed order, two levels.
// Deterministic, no atomics.
#include "message_impl.h"
#include "../../include/maloq_hip.h"

namespace maloq {
namespace rad {

using msg::BF16;
using msg::F32;
using msg::f32x16;
using msg::bf16x8;
using msg::wave_sync;

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
  float* duh;       // backward: [E, c_H] fp32 dL/du_H
  float* dx;        // backward: [E, c0], nullable
  float* part;      // backward partials
  int64_t pstride;  // floats per partial
  int64_t e_per_split;
};

__host__ __device__ constexpr int pitch(int c) { return c + 4; }  // LDS row pitch (floats)

// LDS floats of the staged hidden-layer parameters: per layer W^T [c_i] rows of
// pitch(c_{i+1}) (the staging writes then hit 4-way at most), then bias,
// LayerNorm weight and bias [c_{i+1}].
__host__ __device__ inline int layer_param_floats(int cin, int c) { return cin * pitch(c) + 3 * c; }
__host__ __device__ inline int param_floats(const Args& a) {
  int s = 0;
  for (int i = 0; i < a.nh; ++i) s += layer_param_floats(a.c[i], a.c[i + 1]);
  return s;
}
// Floats of the hidden-layer gradients: per layer dW [c_{i+1}][c_i], db, dgamma, dbeta.
__host__ __device__ inline int grad_floats(const Args& a) {
  int s = 0;
  for (int i = 0; i < a.nh; ++i) s += a.c[i + 1] * (a.c[i] + 3);
  return s;
}

// Floats of the chain kernel's per-wave column sums: per layer [3][8 waves][c_{i+1}].
__host__ __device__ inline int cs_floats(const Args& a) {
  int s = 0;
  for (int i = 0; i < a.nh; ++i) s += 3 * 8 * a.c[i + 1];
  return s;
}

// gfx950 converts two floats to bf16 (round to nearest even) in one instruction.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

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
  f.x = pk_bf16(a.x, a.y);
  f.y = pk_bf16(a.z, a.w);
  f.z = pk_bf16(b.x, b.y);
  f.w = pk_bf16(b.z, b.w);
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


// ---------------------------------------------------------------- staging
// Global -> LDS copies are issued in batches of SB loads (indices clamped in
// range, so every load is unconditional) before any of them is stored: one
// memory latency per batch instead of one per element.
constexpr int SB = 8;
// Hidden-layer parameters into LDS (layout of param_floats); the caller syncs.
template <int NTH>
__device__ __forceinline__ void stage_params(const Args& a, float* prm, int tid) {
  float* p = prm;
  for (int i = 0; i < a.nh; ++i) {
    const int cin = a.c[i], c = a.c[i + 1], n = c * cin;
    const float* W = a.w[i];
    for (int t0 = tid; t0 < n; t0 += NTH * SB) {
      float v[SB];
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int t = t0 + u * NTH;
        v[u] = W[t < n ? t : n - 1];  // coalesced read of W[j][k]
      }
#pragma unroll
      for (int u = 0; u < SB; ++u) {
        const int t = t0 + u * NTH;
        if (t < n) {
          const int j = t / cin, k = t - j * cin;
          p[k * pitch(c) + j] = v[u];
        }
      }
    }
    p += cin * pitch(c);
    for (int t = tid; t < c; t += NTH) {
      const float bv = a.b[i][t], gv = a.g[i][t], tv = a.bt[i][t];
      p[t] = bv;
      p[c + t] = gv;
      p[2 * c + t] = tv;
    }
    p += 3 * c;
  }
}
// n floats -> LDS, batched; the caller syncs.
template <int NTH>
__device__ __forceinline__ void stage_vec(const float* __restrict__ src, int n, float* dst, int tid) {
  for (int i0 = tid; i0 < n; i0 += NTH * SB) {
    float v[SB];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int i = i0 + u * NTH;
      v[u] = src[i < n ? i : n - 1];
    }
#pragma unroll
    for (int u = 0; u < SB; ++u)
      if (i0 + u * NTH < n) dst[i0 + u * NTH] = v[u];
  }
}
// Rows [e0, e0 + TE) of an fp32 [E, w] array into LDS rows of pitch(w), zero
// beyond the last valid edge; the caller syncs.
template <int NTH>
__device__ __forceinline__ void stage_rows(const float* __restrict__ src, int64_t e0, int nvalid, int w,
                                           float* dst, int tid) {
  const int n4 = w >> 2, n = TE * n4;
  for (int i0 = tid; i0 < n; i0 += NTH * 4) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NTH, e = i / n4, k = (i - e * n4) * 4;
      const int er = e < nvalid ? e : nvalid - 1;
      v[u] = *reinterpret_cast<const float4*>(src + (e0 + er) * w + (i < n ? k : 0));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int i = i0 + u * NTH, e = i / n4, k = (i - e * n4) * 4;
      if (i < n) *reinterpret_cast<float4*>(dst + e * pitch(w) + k) = e < nvalid ? v[u] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
}

// ---------------------------------------------------------------- hidden chain
// Logistic function and SiLU with the hardware exp and reciprocal (about 2 ulp).
__device__ __forceinline__ float sigm(float a) { return __builtin_amdgcn_rcpf(1.0f + __expf(-a)); }
__device__ __forceinline__ float silu_f(float a) { return a * sigm(a); }

// fp32 MFMA 32x32x2 (exact fp32 products): lane i supplies A[m = i%32][k = i/32]
// and B[k = i/32][n = i%32]; D lane L register r is (m = 8 (r/4) + 4 (L/32) + r%4,
// n = L%32).
__device__ __forceinline__ void mfma2(f32x16& acc, float a, float b) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Tile GEMM on LDS operands: D[m][n] = sum_k A(m, k) B(k, n) over k < K (K even)
// for the 32 x 32 tile at (m0, n0); A(m, k) = pa[m * sam + k * sak], B(k, n) =
// pb[k * sbk + n * sbn], columns n >= nmax read as 0.  Two accumulators
// (alternate k pairs) keep consecutive MFMAs independent.
// With ACT, B(k, n) = SiLU(gam[n] pb[...] + bet[n]) (an activation recomputed
// from its normalised input).
template <bool ACT = false>
__device__ __forceinline__ f32x16 tile_gemm(const float* pa, int sam, int sak, const float* pb, int sbk,
                                            int sbn, int K, int m0, int n0, int nmax, int lane,
                                            const float* gam = nullptr, const float* bet = nullptr) {
  f32x16 acc0, acc1;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    acc0[r] = 0.f;
    acc1[r] = 0.f;
  }
  const int h = lane >> 5, n = n0 + (lane & 31);
  const float* ap = pa + (m0 + (lane & 31)) * sam + h * sak;
  const bool nok = n < nmax;
  const float* bp = pb + h * sbk + (nok ? n : 0) * sbn;
  float gn = 0.f, bn = 0.f;
  if constexpr (ACT) {
    gn = gam[nok ? n : 0];
    bn = bet[nok ? n : 0];
  }
  auto bval = [&](const float* q) {
    if constexpr (ACT) return nok ? silu_f(fmaf(gn, *q, bn)) : 0.f;
    else return nok ? *q : 0.f;
  };
  int k = 0;
  for (; k + 8 <= K; k += 8) {  // 4 operand pairs in flight
    float av[4], bv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      av[u] = ap[(k + 2 * u) * sak];
      bv[u] = bval(bp + (k + 2 * u) * sbk);
    }
    mfma2(acc0, av[0], bv[0]);
    mfma2(acc1, av[1], bv[1]);
    mfma2(acc0, av[2], bv[2]);
    mfma2(acc1, av[3], bv[3]);
  }
  for (; k < K; k += 2) mfma2(acc0, ap[k * sak], bval(bp + k * sbk));
#pragma unroll
  for (int r = 0; r < 16; ++r) acc0[r] += acc1[r];
  return acc0;
}

// Row statistics across the NW waves: red [2][NW][TE].
template <int NW>
__device__ __forceinline__ float wave_sum(const float* red, int lane) {
  float s = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) s += red[w * TE + lane];
  return s;
}

// One hidden layer for the tile (C outputs, NW waves): z = ain W^T + b on the
// MFMA (32 x 32 tiles round-robin over the waves) into zb [TE][pitch(C)],
// then per lane (= edge) LayerNorm over the row, the wave owning outputs
// [Q wave, Q wave + Q), Q = C / NW: xhat in place in zb, rstd to rs (if
// non-null), u = SiLU(gamma xhat + beta) to aout (if non-null; may be zb).
template <int C, int NW>
__device__ __forceinline__ void hidden_fwd(const float* prm, int cin, const float* ain, float* zb,
                                           float* rs, float* aout, float* red, float eps, int wave,
                                           int lane) {
  constexpr int NNT = C / 32, Q = C / NW;
  static_assert(Q % 4 == 0, "outputs per wave must be a multiple of 4");
  const float* wt = prm;
  const float* bias = prm + pitch(C) * cin;
  const float* gam = bias + C;
  const float* bet = gam + C;
  for (int t = wave; t < 2 * NNT; t += NW) {
    const int m0 = 32 * (t / NNT), n0 = 32 * (t % NNT);
    const f32x16 acc = tile_gemm(ain, pitch(cin), 1, wt, pitch(C), 1, cin, m0, n0, C, lane);
    const int j = n0 + (lane & 31);
    const float bj = bias[j];
#pragma unroll
    for (int r = 0; r < 16; ++r) zb[(m0 + acc_row(r, lane)) * pitch(C) + j] = acc[r] + bj;
  }
  __syncthreads();
  const int j0 = wave * Q;
  float z[Q];
  float s1 = 0.f;
#pragma unroll
  for (int q = 0; q < Q; q += 4) {
    const float4 v = *reinterpret_cast<const float4*>(zb + lane * pitch(C) + j0 + q);
    z[q] = v.x; z[q + 1] = v.y; z[q + 2] = v.z; z[q + 3] = v.w;
    s1 += (v.x + v.y) + (v.z + v.w);
  }
  red[wave * TE + lane] = s1;
  __syncthreads();
  constexpr float inv_c = 1.0f / static_cast<float>(C);
  const float mean = wave_sum<NW>(red, lane) * inv_c;
  float s2 = 0.f;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    z[q] -= mean;
    s2 = fmaf(z[q], z[q], s2);
  }
  red[NW * TE + wave * TE + lane] = s2;
  __syncthreads();
  const float var = wave_sum<NW>(red + NW * TE, lane) * inv_c;
  const float rstd = 1.0f / sqrtf(var + eps);
  if (rs != nullptr && wave == 0) rs[lane] = rstd;
#pragma unroll
  for (int q = 0; q < Q; q += 4) {
    const float4 x4 = make_float4(z[q] * rstd, z[q + 1] * rstd, z[q + 2] * rstd, z[q + 3] * rstd);
    *reinterpret_cast<float4*>(zb + lane * pitch(C) + j0 + q) = x4;
    if (aout != nullptr) {
      const float4 g4 = *reinterpret_cast<const float4*>(gam + j0 + q);
      const float4 t4 = *reinterpret_cast<const float4*>(bet + j0 + q);
      const float4 u = make_float4(silu_f(fmaf(g4.x, x4.x, t4.x)), silu_f(fmaf(g4.y, x4.y, t4.y)),
                                   silu_f(fmaf(g4.z, x4.z, t4.z)), silu_f(fmaf(g4.w, x4.w, t4.w)));
      *reinterpret_cast<float4*>(aout + lane * pitch(C) + j0 + q) = u;
    }
  }
  __syncthreads();  // red reusable; rows complete for every wave
}

template <int NW>
__device__ __forceinline__ void hidden_layer(int c, const float* prm, int cin, const float* ain,
                                             float* zb, float* rs, float* aout, float* red, float eps,
                                             int wave, int lane) {
  switch (c) {
    case 32: hidden_fwd<32, NW>(prm, cin, ain, zb, rs, aout, red, eps, wave, lane); break;
    case 64: hidden_fwd<64, NW>(prm, cin, ain, zb, rs, aout, red, eps, wave, lane); break;
    case 96: hidden_fwd<96, NW>(prm, cin, ain, zb, rs, aout, red, eps, wave, lane); break;
    default: hidden_fwd<128, NW>(prm, cin, ain, zb, rs, aout, red, eps, wave, lane); break;
  }
}

// ---------------------------------------------------------------- forward
// Persistent: each workgroup (FW_W waves) stages the hidden parameters and the
// output bias once, then works through an equal share of the (64-edge tile,
// 128-byte output group) units, in order: for each tile its share touches it
// runs the hidden chain, then its waves split the tile's groups of that share
// (contiguous ranges of 32-output tiles, W_o fragments loaded in chunks of
// MAXT tiles as they are used).  Equal shares of units rather than whole
// tiles: 575 tiles on 256 CUs would give some CUs three tiles against an
// average of 2.25.  Only the workgroup holding a tile's first group saves
// u_H.  The output loop has no loads, so its stores are never waited on.
// Results go through a per-wave LDS block of 64 edges x 128 bytes of outputs
// and leave as whole 128-byte row segments (16 bytes per lane, eight lanes per
// row): stores in the accumulator's lane order (16 bytes per row per
// instruction) reach less than half the HBM write rate.
constexpr int FW_W = 8;
constexpr int FW_SP = 128 + 16;  // bytes per staged row (the pad spreads rows over the banks)
template <class TM, int NNT>
__global__ __launch_bounds__(FW_W * 64) void radial_fwd_kernel(Args a) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  using raw = typename TM::raw;
  constexpr int KC = TM::KC, VEC = TM::VEC, NTH = FW_W * 64;
  constexpr int CH = 32 * NNT, NK = CH / KC, MAXT = (16 / NK) > 0 ? 16 / NK : 1;  // W_o fragment budget
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t ntiles = (a.E + TE - 1) / TE;
  const int cout = a.c[a.nh + 1];
  int cmax = 0;
  for (int i = 1; i <= a.nh; ++i) cmax = a.c[i] > cmax ? a.c[i] : cmax;
  float* red = smem;                          // [2][FW_W][TE]
  float* bo = red + 2 * FW_W * TE;            // [c_out] output bias
  float* prm = bo + cout;                     // staged parameters
  float* act0 = prm + param_floats(a);        // [TE][pitch(c0)]
  float* buf0 = act0 + TE * pitch(a.c[0]);    // [TE][pitch(cmax)] x2: activations
  float* buf1 = buf0 + TE * pitch(cmax);
  char* stg = reinterpret_cast<char*>(buf1 + TE * pitch(cmax)) + wave * TE * FW_SP;  // this wave's block
  stage_vec<NTH>(a.bo, cout, bo, tid);
  stage_params<NTH>(a, prm, tid);
  // this wave's output tiles [tw0, tw0 + ntw) of the current edge tile and
  // their W_o fragments (chunks of MAXT tiles)
  constexpr int GT = 64 / (sizeof(raw) * 16);  // tiles per 128-byte group: 2 (bf16) or 1 (fp32)
  const int not_ = cout / 32, ngrp = not_ / GT;
  int tw0 = 0, ntw = 0;
  const raw* wo = reinterpret_cast<const raw*>(a.wo);
  const raw* wlane = wo + static_cast<int64_t>(lane & 31) * CH + (lane >> 5) * VEC;
  frag_t af[MAXT][NK];
  auto load_chunk = [&](int t0) {
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
      int ot = tw0 + t0 + t;
      ot = ot < not_ ? ot : not_ - 1;  // clamped: every load is unconditional
#pragma unroll
      for (int kc = 0; kc < NK; ++kc)
        af[t][kc] = *reinterpret_cast<const frag_t*>(wlane + static_cast<int64_t>(ot) * 32 * CH + kc * KC);
    }
  };
  __syncthreads();
  raw* out = reinterpret_cast<raw*>(a.out);
  // this workgroup's units [u0, u1) of ntiles x ngrp
  const int64_t units = ntiles * ngrp;
  const int64_t u0 = static_cast<int64_t>(blockIdx.x) * units / gridDim.x;
  const int64_t u1 = static_cast<int64_t>(blockIdx.x + 1) * units / gridDim.x;
  if (u0 >= u1) return;  // whole workgroup
  for (int64_t tile = u0 / ngrp; tile * ngrp < u1; ++tile) {
    const int glo = static_cast<int>(u0 > tile * ngrp ? u0 - tile * ngrp : 0);
    const int ghi = static_cast<int>(u1 - tile * ngrp < ngrp ? u1 - tile * ngrp : ngrp);
    {
      const int n = ghi - glo, gw0 = glo + wave * n / FW_W, gw1 = glo + (wave + 1) * n / FW_W;
      tw0 = gw0 * GT;
      ntw = (gw1 - gw0) * GT;
    }
    const int64_t e0 = tile * TE;
    const int nvalid = static_cast<int>((a.E - e0) < TE ? (a.E - e0) : TE);
    stage_rows<NTH>(a.x, e0, nvalid, a.c[0], act0, tid);
    __syncthreads();
    const float* ain = act0;
    {
      const float* p = prm;
      float* cur = buf0;
      for (int i = 0; i < a.nh; ++i) {
        hidden_layer<FW_W>(a.c[i + 1], p, a.c[i], ain, cur, nullptr, cur, red, a.eps, wave, lane);
        p += layer_param_floats(a.c[i], a.c[i + 1]);
        ain = cur;
        cur = (cur == buf0) ? buf1 : buf0;
      }
    }
    const float* uH = ain;  // [TE][pitch(CH)]
    // saved u_H rows (TM raw) for the weight gradient: the CH / VEC 16-byte
    // pieces of each row round-robin over the waves
    if (a.save != nullptr && glo == 0 && lane < nvalid) {
      raw* sv = reinterpret_cast<raw*>(a.save) + (e0 + lane) * CH;
      for (int f = wave; f < CH / VEC; f += FW_W)
        *reinterpret_cast<frag_t*>(sv + f * VEC) = pack_frag(uH + lane * pitch(CH) + f * VEC, TM{});
    }
    // B fragments: u_H^T, lane (edge 32 nt + lane % 32, K half lane / 32)
    frag_t bf[2][NK];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int kc = 0; kc < NK; ++kc)
        bf[nt][kc] = pack_frag(uH + (32 * nt + (lane & 31)) * pitch(CH) + kc * KC + (lane >> 5) * VEC, TM{});
    for (int t0 = 0; t0 < ntw; t0 += MAXT) {
      load_chunk(t0);
#pragma unroll
      for (int t = 0; t < MAXT; ++t) {
        if (t0 + t >= ntw) break;
        const int ot = tw0 + t0 + t, gt = (t0 + t) % GT;  // tile within its 128-byte group
        f32x16 acc[2];
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[nt][r] = 0.f;
#pragma unroll
        for (int kc = 0; kc < NK; ++kc) {
          mfma(acc[0], af[t][kc], bf[0][kc], TM{});
          mfma(acc[1], af[t][kc], bf[1][kc], TM{});
        }
        // lane L, register r: output ot 32 + 8 (r/4) + 4 (L/32) + r%4, edge 32 nt + L%32
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          const int e = 32 * nt + (lane & 31);
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int ol = 8 * g4 + 4 * (lane >> 5);  // output within the tile
            const float4 bb = *reinterpret_cast<const float4*>(bo + ot * 32 + ol);
            const float v0 = acc[nt][4 * g4] + bb.x, v1 = acc[nt][4 * g4 + 1] + bb.y;
            const float v2 = acc[nt][4 * g4 + 2] + bb.z, v3 = acc[nt][4 * g4 + 3] + bb.w;
            char* d = stg + e * FW_SP + (gt * 32 + ol) * static_cast<int>(sizeof(raw));
            if constexpr (sizeof(raw) == 2)
              *reinterpret_cast<uint2*>(d) = make_uint2(pk_bf16(v0, v1), pk_bf16(v2, v3));
            else
              *reinterpret_cast<float4*>(d) = make_float4(v0, v1, v2, v3);
          }
        }
        if (gt == GT - 1) {  // group complete: 64 rows x 128 bytes, 8 lanes per row
          wave_sync();
          const int64_t col = static_cast<int64_t>(ot - (GT - 1)) * 32;  // first output of the group
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int e = 8 * i + (lane >> 3), ch = lane & 7;
            const uint4 v = *reinterpret_cast<const uint4*>(stg + e * FW_SP + ch * 16);
            if (e < nvalid)
              *reinterpret_cast<uint4*>(reinterpret_cast<char*>(out + (e0 + e) * cout + col) + ch * 16) = v;
          }
          wave_sync();
        }
      }
    }
    __syncthreads();  // LDS rows of this tile read by every wave
  }
}

// ---------------------------------------------------------------- backward
// du_H [e][j] = sum_o G[e][o] W_o[o][j] for du_te<NNT>() = 32 du_rt<NNT>()
// edges per workgroup (each W_o fragment serves du_rt row tiles: 2 for
// c_H <= 64, else 1 within the register budget).  Wave w of DU_W takes
// 1/DU_W of the K (output) range for all DU_RT x NNT tiles; its A (G rows) and
// B (W_o^T rows) fragments of up to DU_KS steps are all in flight before the
// first wait, then the MFMAs run; the partial tiles are summed by a fixed
// three-level tree through LDS (waves w and w + 4, then w and w + 2, then 0
// and 1).
constexpr int DU_W = 8;
template <int NNT>
__host__ __device__ constexpr int du_rt() { return NNT <= 2 ? 2 : 1; }
template <int NNT>
__host__ __device__ constexpr int du_te() { return 32 * du_rt<NNT>(); }
template <class TM, int NNT>
__global__ __launch_bounds__(DU_W * 64) void radial_du_kernel(Args a) {
  constexpr int CH = 32 * NNT, KC = TM::KC, VEC = TM::VEC;
  constexpr int DU_RT = du_rt<NNT>(), DU_TE = du_te<NNT>();
  constexpr int DU_KS = 6;  // steps in flight (register budget)
  constexpr int SLOT = DU_TE * pitch(CH);
  __shared__ alignas(16) float red[4 * SLOT];
  using raw = typename TM::raw;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * DU_TE;
  const int nvalid = static_cast<int>((a.E - e0) < DU_TE ? (a.E - e0) : DU_TE);
  const int cout = a.c[a.nh + 1];
  const raw* G = reinterpret_cast<const raw*>(a.grad);
  const raw* wot = reinterpret_cast<const raw*>(a.wot);
  const int nks = cout / KC, ks0 = wave * nks / DU_W, kq = (wave + 1) * nks / DU_W - ks0;
  const raw* ga[DU_RT];
#pragma unroll
  for (int rt = 0; rt < DU_RT; ++rt) {
    int e = 32 * rt + (lane & 31);
    e = e < nvalid ? e : nvalid - 1;  // in-bounds rows; results of padded edges are not stored
    ga[rt] = G + (e0 + e) * cout + (lane >> 5) * VEC + ks0 * KC;
  }
  const raw* gb = wot + static_cast<int64_t>(lane & 31) * cout + (lane >> 5) * VEC + ks0 * KC;
  f32x16 acc[DU_RT][NNT];
#pragma unroll
  for (int rt = 0; rt < DU_RT; ++rt)
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[rt][nt][r] = 0.f;
  for (int c0 = 0; c0 < kq; c0 += DU_KS) {
    frag_t fa[DU_KS][DU_RT], fb[DU_KS][NNT];
#pragma unroll
    for (int s = 0; s < DU_KS; ++s) {
      const int st = c0 + s < kq ? c0 + s : kq - 1;  // clamped: every load is unconditional
#pragma unroll
      for (int rt = 0; rt < DU_RT; ++rt) fa[s][rt] = *reinterpret_cast<const frag_t*>(ga[rt] + st * KC);
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
        fb[s][nt] = *reinterpret_cast<const frag_t*>(gb + static_cast<int64_t>(32 * nt) * cout + st * KC);
    }
#pragma unroll
    for (int s = 0; s < DU_KS; ++s)
      if (c0 + s < kq)
#pragma unroll
        for (int rt = 0; rt < DU_RT; ++rt)
#pragma unroll
          for (int nt = 0; nt < NNT; ++nt) mfma(acc[rt][nt], fa[s][rt], fb[s][nt], TM{});
  }
  // lane L, register r of row tile rt -> edge 32 rt + 8 (r/4) + 4 (L/32) + r%4,
  // column 32 nt + L%32
  auto put = [&](float* slot) {
#pragma unroll
    for (int rt = 0; rt < DU_RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          slot[(32 * rt + acc_row(r, lane)) * pitch(CH) + 32 * nt + (lane & 31)] = acc[rt][nt][r];
  };
  auto add = [&](const float* slot) {
#pragma unroll
    for (int rt = 0; rt < DU_RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          acc[rt][nt][r] += slot[(32 * rt + acc_row(r, lane)) * pitch(CH) + 32 * nt + (lane & 31)];
  };
  if (wave >= 4) put(red + (wave - 4) * SLOT);
  __syncthreads();
  if (wave < 4) add(red + wave * SLOT);
  __syncthreads();
  if (wave == 2 || wave == 3) put(red + (wave - 2) * SLOT);
  __syncthreads();
  if (wave < 2) add(red + wave * SLOT);
  __syncthreads();
  if (wave == 1) put(red);
  __syncthreads();
  if (wave == 0) {
    add(red);
    // lane L writes column 32 nt + L%32 of rows 32 rt + acc_row(r, L)
#pragma unroll
    for (int rt = 0; rt < DU_RT; ++rt)
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int ee = 32 * rt + acc_row(r, lane);
          if (ee < nvalid) a.duh[(e0 + ee) * CH + 32 * nt + (lane & 31)] = acc[rt][nt][r];
        }
  }
}

// Backward of hidden layer i for the tile (lane = edge, the wave's Q = C / NW
// of the C outputs): du (LDS rows, pitch(C)) holds dL/du_i on entry and da on
// exit; dz gets dL/dz_i (pre-LayerNorm).
template <int C, int NW>
__device__ __forceinline__ void layer_bwd(const float* prm, int cin, const float* xh, float rstd,
                                          float* du, float* dz, float* red, bool valid, int wave,
                                          int lane) {
  constexpr int Q = C / NW;
  const float* gam = prm + pitch(C) * cin + C;
  const float* bet = gam + C;
  const int j0 = wave * Q;
  const float* xr = xh + lane * pitch(C) + j0;
  float* dur = du + lane * pitch(C) + j0;
  float* dzr = dz + lane * pitch(C) + j0;
  float xv[Q], dh[Q];
  float s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int q = 0; q < Q; q += 4) {
    const float4 x4 = *reinterpret_cast<const float4*>(xr + q);
    const float4 d4 = *reinterpret_cast<const float4*>(dur + q);
    const float4 g4 = *reinterpret_cast<const float4*>(gam + j0 + q);
    const float4 t4 = *reinterpret_cast<const float4*>(bet + j0 + q);
    const float xs[4] = {x4.x, x4.y, x4.z, x4.w}, ds[4] = {d4.x, d4.y, d4.z, d4.w};
    const float gs[4] = {g4.x, g4.y, g4.z, g4.w}, ts[4] = {t4.x, t4.y, t4.z, t4.w};
    float da[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float av = fmaf(gs[t], xs[t], ts[t]);
      const float sg = sigm(av);
      da[t] = valid ? ds[t] * (sg * (1.0f + av * (1.0f - sg))) : 0.f;
      xv[q + t] = xs[t];
      dh[q + t] = da[t] * gs[t];
      s1 += dh[q + t];
      s2 = fmaf(dh[q + t], xs[t], s2);
    }
    *reinterpret_cast<float4*>(dur + q) = make_float4(da[0], da[1], da[2], da[3]);
  }
  red[wave * TE + lane] = s1;
  red[NW * TE + wave * TE + lane] = s2;
  __syncthreads();
  constexpr float inv_c = 1.0f / static_cast<float>(C);
  const float m1 = wave_sum<NW>(red, lane) * inv_c;
  const float m2 = wave_sum<NW>(red + NW * TE, lane) * inv_c;
#pragma unroll
  for (int q = 0; q < Q; q += 4) {
    float4 h;
    h.x = rstd * (dh[q] - m1 - xv[q] * m2);
    h.y = rstd * (dh[q + 1] - m1 - xv[q + 1] * m2);
    h.z = rstd * (dh[q + 2] - m1 - xv[q + 2] * m2);
    h.w = rstd * (dh[q + 3] - m1 - xv[q + 3] * m2);
    *reinterpret_cast<float4*>(dzr + q) = h;
  }
}

template <int NW>
__device__ __forceinline__ void layer_backward(int c, const float* prm, int cin, const float* xh, float rstd,
                                               float* du, float* dz, float* red, bool valid, int wave,
                                               int lane) {
  switch (c) {
    case 32: layer_bwd<32, NW>(prm, cin, xh, rstd, du, dz, red, valid, wave, lane); break;
    case 64: layer_bwd<64, NW>(prm, cin, xh, rstd, du, dz, red, valid, wave, lane); break;
    case 96: layer_bwd<96, NW>(prm, cin, xh, rstd, du, dz, red, valid, wave, lane); break;
    default: layer_bwd<128, NW>(prm, cin, xh, rstd, du, dz, red, valid, wave, lane); break;
  }
}

// Persistent: each workgroup (CW_W waves) stages the hidden parameters once,
// then loops over 64-edge tiles; the weight-gradient tiles and the per-wave
// column sums accumulate in LDS (each element owned by one wave), and the
// workgroup writes one partial at the end.
constexpr int CW_W = 8;
__global__ __launch_bounds__(CW_W * 64) void radial_chain_kernel(Args a) {
  static_assert(CW_W == 8, "cs_floats counts 8 waves");
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int NTH = CW_W * 64;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t ntiles = (a.E + TE - 1) / TE;
  const int nh = a.nh, cH = a.c[nh];
  int cmax = a.c[0];
  for (int i = 1; i <= nh; ++i) cmax = a.c[i] > cmax ? a.c[i] : cmax;
  // LDS regions as offsets from smem (pointers formed at each use keep the
  // accesses in the LDS address space)
  const int o_red = 0;                              // [3][CW_W][TE]
  const int o_rs = o_red + 3 * CW_W * TE;           // [MAXH][TE] rstd per layer
  const int o_dw = o_rs + MAXH * TE;                // weight-gradient accumulators
  const int o_cs = o_dw + grad_floats(a);           // column sums [layer][3][CW_W][c_i]
  const int o_prm = o_cs + cs_floats(a);            // staged parameters
  const int o_act0 = o_prm + param_floats(a);       // [TE][pitch(c0)]
  const int o_xh0 = o_act0 + TE * pitch(a.c[0]);    // [TE][pitch(c_i)] xhat per layer
  auto xh_off = [&](int i) {
    int o = o_xh0;
    for (int k = 0; k < i; ++k) o += TE * pitch(a.c[k + 1]);
    return o;
  };
  auto prm_off = [&](int i) {
    int o = o_prm;
    for (int k = 0; k < i; ++k) o += layer_param_floats(a.c[k], a.c[k + 1]);
    return o;
  };
  auto cs_off = [&](int i) {
    int o = o_cs;
    for (int k = 0; k < i; ++k) o += 3 * CW_W * a.c[k + 1];
    return o;
  };
  auto grad_off = [&](int i) {  // dW_i, db_i, dgamma_i, dbeta_i of layer i
    int o = 0;
    for (int k = 0; k < i; ++k) o += a.c[k + 1] * (a.c[k] + 3);
    return o;
  };
  const int o_du = xh_off(nh);                      // [TE][pitch(cmax)]
  const int o_dz = o_du + TE * pitch(cmax);
  float* red = smem + o_red;
  float* du = smem + o_du;
  float* dz = smem + o_dz;
  float* act0 = smem + o_act0;
  float* dwl = smem + o_dw;
  stage_params<NTH>(a, smem + o_prm, tid);
  for (int i = tid; i < grad_floats(a) + cs_floats(a); i += NTH) dwl[i] = 0.f;  // dW and column sums
  // running column sums: thread (wave, lane) covers edges [8 wave, 8 wave + 8)
  // of columns lane and lane + 64 of each layer
  constexpr int EW = TE / CW_W;
  __syncthreads();
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t e0 = tile * TE;
    const int nvalid = static_cast<int>((a.E - e0) < TE ? (a.E - e0) : TE);
    const bool valid = lane < nvalid;
    stage_rows<NTH>(a.x, e0, nvalid, a.c[0], act0, tid);
    __syncthreads();
    // recompute the chain: xhat and rstd of every layer (activations ping-pong
    // through du and dz, both free until the backward starts)
    {
      const float* ain = act0;
      for (int i = 0; i < nh; ++i) {
        float* aout = (i + 1 < nh) ? ((i & 1) ? dz : du) : nullptr;
        hidden_layer<CW_W>(a.c[i + 1], smem + prm_off(i), a.c[i], ain, smem + xh_off(i), smem + o_rs + i * TE,
                           aout, red, a.eps, wave, lane);
        ain = aout;
      }
    }
    stage_rows<NTH>(a.duh, e0, nvalid, cH, du, tid);
    __syncthreads();
    for (int i = nh - 1; i >= 0; --i) {
      const int c = a.c[i + 1], cin = a.c[i];
      const float* xhi = smem + xh_off(i);
      const float* prm = smem + prm_off(i);
      layer_backward<CW_W>(c, prm, cin, xhi, smem[o_rs + i * TE + lane], du, dz, red, valid, wave, lane);
      __syncthreads();
      // column sums (db, dgamma, dbeta) of this thread's 8 edges
      {
        float* csl = smem + cs_off(i);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int j = lane + 64 * h;
          if (j < c) {
            float sb = 0.f, sg = 0.f, st = 0.f;
#pragma unroll
            for (int e = wave * EW; e < wave * EW + EW; ++e) {
              const float dav = du[e * pitch(c) + j];
              sb += dz[e * pitch(c) + j];
              sg = fmaf(dav, xhi[e * pitch(c) + j], sg);
              st += dav;
            }
            csl[wave * c + j] += sb;
            csl[CW_W * c + wave * c + j] += sg;
            csl[2 * CW_W * c + wave * c + j] += st;
          }
        }
      }
      // dW_i [j][k] += sum_e dz[e][j] u[e][k]: 32 x 32 MFMA tiles over the waves
      // (K = the tile's 64 edges; rows of padded edges are zero in dz); for
      // i > 0, u = SiLU(gamma xhat + beta) of layer i - 1, formed as it is read
      {
        float* dwi = dwl + grad_off(i);
        const int nmt = c / 32, nnt = (cin + 31) / 32;
        for (int t = wave; t < nmt * nnt; t += CW_W) {
          const int m0 = 32 * (t / nnt), n0 = 32 * (t % nnt);
          f32x16 acc;
          if (i > 0) {
            const float* gp = smem + prm_off(i - 1) + pitch(cin) * a.c[i - 1] + cin;
            acc = tile_gemm<true>(dz, 1, pitch(c), smem + xh_off(i - 1), pitch(cin), 1, TE, m0, n0, cin, lane,
                                  gp, gp + cin);
          } else {
            acc = tile_gemm(dz, 1, pitch(c), act0, pitch(cin), 1, TE, m0, n0, cin, lane);
          }
          const int k = n0 + (lane & 31);
          if (k < cin) {
#pragma unroll
            for (int r = 0; r < 16; ++r) dwi[(m0 + acc_row(r, lane)) * cin + k] += acc[r];
          }
        }
      }
      __syncthreads();  // du / red free again
      // du_{i-1} [e][k] = sum_j dz[e][j] W_i[j][k] (W_i^T staged as [k][j]) on the
      // MFMA, into du, or dx for the input
      if (i > 0 || a.dx != nullptr) {
        const int nnt = (cin + 31) / 32;
        for (int t = wave; t < 2 * nnt; t += CW_W) {
          const int m0 = 32 * (t / nnt), n0 = 32 * (t % nnt);
          const f32x16 acc = tile_gemm(dz, pitch(c), 1, prm, 1, pitch(c), c, m0, n0, cin, lane);
          const int k = n0 + (lane & 31);
          if (k < cin) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int e = m0 + acc_row(r, lane);
              if (i > 0)
                du[e * pitch(cin) + k] = acc[r];
              else if (e < nvalid)
                a.dx[(e0 + e) * cin + k] = acc[r];
            }
          }
        }
        __syncthreads();
      }
    }
  }
  // the workgroup's partial: dW_i from LDS, column sums combined in wave order
  __syncthreads();
  float* part = a.part + static_cast<int64_t>(blockIdx.x) * a.pstride;
  for (int i = 0; i < nh; ++i) {
    const int c = a.c[i + 1], cin = a.c[i];
    float* pw = part + grad_off(i);
    const float* dwi = dwl + grad_off(i);
    for (int t = tid; t < c * cin; t += NTH) pw[t] = dwi[t];
    const float* csl = smem + cs_off(i);
    for (int t = tid; t < 3 * c; t += NTH) {
      const int q = t / c, j = t - q * c;
      float v = 0.f;
      for (int w = 0; w < CW_W; ++w) v += csl[q * CW_W * c + w * c + j];
      pw[c * cin + t] = v;
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
constexpr int DO_KB = 8;    // fp32: two-edge MFMA steps per register batch

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

// fp32, NNT = c_H / 32 column tiles of u_H.
template <int NNT>
__global__ __launch_bounds__(NT) void radial_dwo_f32_kernel(Args a) {
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
  constexpr int nnt = NNT;
  f32x16 acc[NNT];
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int nt = 0; nt < NNT; ++nt) acc[nt][r] = 0.f;
  // db_o on the VALU: this lane's running sum of G[e][o] over its half of the
  // edges (even edges for lanes 0-31, odd for 32-63), the halves added at the
  // end.  (An MFMA against a ones column would spend a third of the kernel's
  // MFMA issue on a column sum.)
  float colsum = 0.f;
  const int h = lane >> 5;
  // DO_KB two-edge MFMA steps per batch; the loads of the next batch are in
  // flight while the MFMAs of this one run (two register buffers)
  float av[2][DO_KB], bv[2][DO_KB][NNT];
  auto load = [&](int buf, int64_t e0) {
#pragma unroll
    for (int k = 0; k < DO_KB; ++k) {
      const int64_t er = e0 + 2 * k + h;
      const bool ok = er < ee;
      av[buf][k] = ok ? G[er * cout + o] : 0.f;
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
        bv[buf][k][nt] = (ok && nt < nnt) ? U[er * cH + 32 * nt + (lane & 31)] : 0.f;
    }
  };
  auto step = [&](int buf) {
#pragma unroll
    for (int k = 0; k < DO_KB; ++k) {
      colsum += av[buf][k];
#pragma unroll
      for (int nt = 0; nt < NNT; ++nt)
        if (nt < nnt) acc[nt] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[buf][k], bv[buf][k][nt], acc[nt], 0, 0, 0);
    }
  };
  constexpr int64_t BE = 2 * DO_KB;  // edges per batch
  const int64_t nb = ee > eb ? (ee - eb + BE - 1) / BE : 0;
  if (nb > 0) load(0, eb);
  for (int64_t b = 0; b < nb; b += 2) {
    if (b + 1 < nb) load(1, eb + (b + 1) * BE);
    step(0);
    if (b + 1 < nb) {
      if (b + 2 < nb) load(0, eb + (b + 2) * BE);
      step(1);
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
  }
  // lanes L and L + 32 hold the two halves of output ob + L % 32
  const float other = __shfl_xor(colsum, 32);
  if (h == 0) part[static_cast<int64_t>(cout) * cH + o] = colsum + other;
}

// Fixed-order sums of nparts partial vectors (stride floats apart).  First
// level: consecutive groups of at most RGROUP parts, all loads of a group in
// flight at once -> tmp[g][k].  Second level: the groups in order.
constexpr int RGROUP = 32;
__global__ void radial_reduce1_kernel(const float* __restrict__ part, int64_t n, int64_t nparts,
                                      int64_t stride, float* __restrict__ tmp) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t g = blockIdx.y;
  if (k >= n) return;
  const int64_t p0 = g * RGROUP;
  const int np = static_cast<int>((nparts - p0) < RGROUP ? (nparts - p0) : RGROUP);
  float v[RGROUP];
#pragma unroll
  for (int t = 0; t < RGROUP; ++t) v[t] = t < np ? part[(p0 + t) * stride + k] : 0.f;
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < RGROUP; ++t) s += v[t];
  tmp[g * n + k] = s;
}

__global__ void radial_reduce2_kernel(const float* __restrict__ tmp, int64_t n, int ng,
                                      float* __restrict__ out0, int64_t n0, float* __restrict__ out1) {
  const int64_t k = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (k >= n) return;
  float s = 0.f;
  int g = 0;
  for (; g + 8 <= ng; g += 8) {
    float v[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) v[t] = tmp[(g + t) * n + k];
#pragma unroll
    for (int t = 0; t < 8; ++t) s += v[t];
  }
  for (; g < ng; ++g) s += tmp[g * n + k];
  if (k < n0)
    out0[k] = s;
  else
    out1[k - n0] = s;
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

static int cmax_of(const Args& a, bool with_input) {
  int m = with_input ? a.c[0] : 0;
  for (int i = 1; i <= a.nh; ++i) m = a.c[i] > m ? a.c[i] : m;
  return m;
}
static int64_t fwd_lds(const Args& a) {
  return 4 * (2 * FW_W * TE + a.c[a.nh + 1] + param_floats(a) +
              static_cast<int64_t>(TE) * (pitch(a.c[0]) + 2 * pitch(cmax_of(a, false)))) +
         static_cast<int64_t>(FW_W) * TE * FW_SP;
}
static int64_t chain_lds(const Args& a) {
  int64_t f = 3 * CW_W * TE + MAXH * TE + grad_floats(a) + cs_floats(a) + param_floats(a) +
              static_cast<int64_t>(TE) * pitch(a.c[0]);
  for (int i = 1; i <= a.nh; ++i) f += static_cast<int64_t>(TE) * pitch(a.c[i]);
  f += 2 * static_cast<int64_t>(TE) * pitch(cmax_of(a, true));
  return 4 * f;
}
static int64_t hidden_grad_floats(const Args& a) { return grad_floats(a); }
static int dwo_splits(const Args& a) {
  const int not_ = (a.c[a.nh + 1] + DO_T - 1) / DO_T;
  int s = 512 / not_;
  const int64_t smax = (a.E + 255) / 256;  // at least 256 edges per split
  if (s > smax) s = static_cast<int>(smax);
  return s < 1 ? 1 : (s > 128 ? 128 : s);
}
static int64_t ntiles_of(int64_t E) { return (E + TE - 1) / TE; }
// Workgroups of the persistent kernels: one per compute unit, at most one per tile.
static int persistent_grid(int64_t ntiles) {
  const int cus = device_cus();
  return static_cast<int>(ntiles < cus ? ntiles : cus);
}
static int rgroups(int64_t nparts) { return static_cast<int>((nparts + RGROUP - 1) / RGROUP); }

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
  MALOQ_REQUIRE(chain_lds(a) <= LDS_MAX, "RadialMLP widths need %lld bytes of LDS per workgroup (max %d)",
                static_cast<long long>(chain_lds(a)), LDS_MAX);
  return MALOQ_OK;
}

static int set_params(Args& a, const float* const* w, const float* const* b, const float* const* g,
                      const float* const* bt, float eps) {
  MALOQ_REQUIRE(w && b && g && bt, "null parameter array");
  for (int i = 0; i < a.nh; ++i) {
    MALOQ_REQUIRE(w[i] && b[i] && g[i] && bt[i], "null parameter of hidden layer %d", i);
    a.w[i] = w[i];
    a.b[i] = b[i];
    a.g[i] = g[i];
    a.bt[i] = bt[i];
  }
  MALOQ_REQUIRE(eps > 0.f, "eps must be positive");
  a.eps = eps;
  return MALOQ_OK;
}

template <class TM>
static int launch_fwd(const Args& a, int64_t ntiles, hipStream_t s) {
  const size_t lds = static_cast<size_t>(fwd_lds(a));
  const void* fn = nullptr;
  switch (a.c[a.nh] / 32) {
    case 1: fn = reinterpret_cast<const void*>(&radial_fwd_kernel<TM, 1>); break;
    case 2: fn = reinterpret_cast<const void*>(&radial_fwd_kernel<TM, 2>); break;
    case 3: fn = reinterpret_cast<const void*>(&radial_fwd_kernel<TM, 3>); break;
    default: fn = reinterpret_cast<const void*>(&radial_fwd_kernel<TM, 4>); break;
  }
  int rc = dyn_lds(fn, lds);
  if (rc) return rc;
  const dim3 grid(static_cast<unsigned>(persistent_grid(ntiles))), block(FW_W * 64);
  switch (a.c[a.nh] / 32) {
    case 1: hipLaunchKernelGGL((radial_fwd_kernel<TM, 1>), grid, block, lds, s, a); break;
    case 2: hipLaunchKernelGGL((radial_fwd_kernel<TM, 2>), grid, block, lds, s, a); break;
    case 3: hipLaunchKernelGGL((radial_fwd_kernel<TM, 3>), grid, block, lds, s, a); break;
    default: hipLaunchKernelGGL((radial_fwd_kernel<TM, 4>), grid, block, lds, s, a); break;
  }
  return check_launch("radial_fwd_kernel");
}

template <class TM>
static int launch_du(const Args& a, int64_t ntiles, hipStream_t s) {
  (void)ntiles;
  const dim3 block(DU_W * 64);
  auto grid = [&](int te) { return dim3(static_cast<unsigned>((a.E + te - 1) / te)); };
  switch (a.c[a.nh] / 32) {
    case 1: hipLaunchKernelGGL((radial_du_kernel<TM, 1>), grid(du_te<1>()), block, 0, s, a); break;
    case 2: hipLaunchKernelGGL((radial_du_kernel<TM, 2>), grid(du_te<2>()), block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((radial_du_kernel<TM, 3>), grid(du_te<3>()), block, 0, s, a); break;
    default: hipLaunchKernelGGL((radial_du_kernel<TM, 4>), grid(du_te<4>()), block, 0, s, a); break;
  }
  return check_launch("radial_du_kernel");
}

// Fixed-order sum of nparts partial vectors of n floats (stride apart) into
// out0 [0, n0) and out1 [n0, n); tmp holds rgroups(nparts) x n floats.
static int reduce(const float* part, int64_t n, int64_t nparts, int64_t stride, float* tmp, float* out0,
                  int64_t n0, float* out1, hipStream_t s) {
  const int ng = rgroups(nparts);
  const unsigned nb = static_cast<unsigned>((n + 255) / 256);
  hipLaunchKernelGGL(radial_reduce1_kernel, dim3(nb, ng), dim3(256), 0, s, part, n, nparts, stride, tmp);
  int rc = check_launch("radial_reduce1_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(radial_reduce2_kernel, dim3(nb), dim3(256), 0, s, static_cast<const float*>(tmp), n, ng,
                     out0, n0, out1);
  return check_launch("radial_reduce2_kernel");
}

extern "C" int64_t maloq_radial_pack_bytes(int dtype, int c_out, int c_hidden) {
  if (dtype != 0 && dtype != 1) return -1;
  return 2 * static_cast<int64_t>(c_out) * c_hidden * (dtype == 1 ? 2 : 4);
}

extern "C" int64_t maloq_radial_bwd_partials_floats(int dtype, int nhidden, const int* widths,
                                                    int64_t num_edges) {
  Args a;
  if (setup(a, dtype, nhidden, widths, num_edges)) return -1;
  const int64_t nt = ntiles_of(num_edges);
  const int cH = a.c[a.nh], cout = a.c[a.nh + 1];
  const int64_t ph = hidden_grad_floats(a), po = static_cast<int64_t>(cout) * cH + cout;
  const int64_t h = num_edges * cH + (nt + rgroups(nt)) * ph;
  const int sp = dwo_splits(a);
  const int64_t o = (sp + rgroups(sp)) * po;
  return (h > o ? h : o) + 4;
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
  MALOQ_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(save) & 15) == 0, "x / out / save must be 16-byte aligned");
  a.x = x;
  a.wo = wo;
  a.wot = wot;
  a.bo = out_bias;
  a.out = out;
  a.save = save;
  const int64_t ntiles = ntiles_of(num_edges);
  MALOQ_REQUIRE(ntiles < (int64_t(1) << 31), "too many edges");
  return dtype == 1 ? launch_fwd<BF16>(a, ntiles, s) : launch_fwd<F32>(a, ntiles, s);
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
  MALOQ_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(grad) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(save) & 15) == 0 && (reinterpret_cast<uintptr_t>(partials) & 15) == 0 &&
                (reinterpret_cast<uintptr_t>(grad_x) & 15) == 0, "buffers must be 16-byte aligned");
  const int cH = a.c[a.nh], cout = a.c[a.nh + 1];
  const size_t el = dtype == 1 ? 2 : 4;
  a.x = x;
  a.wo = wpack;
  a.wot = static_cast<const char*>(wpack) + static_cast<size_t>(cout) * cH * el;
  a.grad = grad;
  a.save = const_cast<void*>(save);  // read-only in the backward
  a.dx = grad_x;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t ntiles = ntiles_of(num_edges);
  MALOQ_REQUIRE(ntiles < (int64_t(1) << 31), "too many edges");
  // workspace: dL/du_H [E, c_H], per-tile hidden partials, first-level sums
  a.duh = partials;
  rc = dtype == 1 ? launch_du<BF16>(a, ntiles, s) : launch_du<F32>(a, ntiles, s);
  if (rc) return rc;
  const int64_t ph = hidden_grad_floats(a);
  a.part = partials + num_edges * cH;
  a.pstride = ph;
  const size_t lds = static_cast<size_t>(chain_lds(a));
  rc = dyn_lds(reinterpret_cast<const void*>(&radial_chain_kernel), lds);
  if (rc) return rc;
  const int cgrid = persistent_grid(ntiles);
  hipLaunchKernelGGL(radial_chain_kernel, dim3(static_cast<unsigned>(cgrid)), dim3(CW_W * 64), lds, s, a);
  rc = check_launch("radial_chain_kernel");
  if (rc) return rc;
  rc = reduce(a.part, ph, cgrid, ph, a.part + static_cast<int64_t>(cgrid) * ph, grad_hidden, ph, grad_hidden, s);
  if (rc) return rc;
  // output layer: split-K partials of [dW_o | db_o] (the workspace is reused:
  // stream order puts this after the sums above), then their sum
  const int splits = dwo_splits(a);
  a.e_per_split = ((num_edges + splits - 1) / splits + DO_KE - 1) / DO_KE * DO_KE;
  const int64_t po = static_cast<int64_t>(cout) * cH + cout;
  a.part = partials;
  a.pstride = po;
  const int not_ = (cout + DO_T - 1) / DO_T;
  if (dtype == 1)
    hipLaunchKernelGGL(radial_dwo_kernel<BF16>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a);
  else
    switch (a.c[a.nh] / 32) {
      case 1: hipLaunchKernelGGL(radial_dwo_f32_kernel<1>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a); break;
      case 2: hipLaunchKernelGGL(radial_dwo_f32_kernel<2>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a); break;
      case 3: hipLaunchKernelGGL(radial_dwo_f32_kernel<3>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a); break;
      default: hipLaunchKernelGGL(radial_dwo_f32_kernel<4>, dim3(static_cast<unsigned>(not_ * splits)), dim3(NT), 0, s, a); break;
    }
  rc = check_launch("radial_dwo_kernel");
  if (rc) return rc;
  return reduce(partials, po, splits, po, partials + splits * po, grad_out_weight,
                static_cast<int64_t>(cout) * cH, grad_out_bias, s);
}
