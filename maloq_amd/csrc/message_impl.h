#pragma once
// Shared device code of the fused equivariant message block on gfx950: operand
// types, the compile-time plan of kept rows (|m| <= mmax) and Wigner entries,
// kernel arguments, and the per-edge prep kernel (Wigner rows + rotation into
// the edge frame).  The SO(2) GEMM with its inverse-rotation / segment-sum
// epilogue is in message_gemm.h.
#include <type_traits>
#include <utility>

#include "common.h"
#include "wigner_device.h"

namespace maloq {
namespace msg {

constexpr int CB = 32;      // output channels per workgroup
constexpr int FRAG = 1024;  // bytes per MFMA operand fragment in LDS

typedef short bf16x8 __attribute__((__vector_size__(8 * sizeof(short))));
typedef float f32x4 __attribute__((__vector_size__(4 * sizeof(float))));
typedef float f32x16 __attribute__((__vector_size__(16 * sizeof(float))));

struct BF16 {
  using raw = uint16_t;
  static constexpr int KC = 16;  // channels per K step (one fragment)
  static constexpr int VEC = 8;  // elements per 16-byte lane load
  static __device__ __forceinline__ float load(const raw* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ raw cvt(float v) { return f32_to_bf16(v); }
};
struct F32 {
  using raw = float;
  static constexpr int KC = 8;
  static constexpr int VEC = 4;
  static __device__ __forceinline__ float load(const raw* p) { return *p; }
  static __device__ __forceinline__ raw cvt(float v) { return v; }
};

__device__ __forceinline__ void mma(f32x16& acc, const char* a, const char* b, int lane, BF16) {
  const bf16x8 av = *reinterpret_cast<const bf16x8*>(a + lane * 16);
  const bf16x8 bv = *reinterpret_cast<const bf16x8*>(b + lane * 16);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x16& acc, const char* a, const char* b, int lane, F32) {
  const f32x4 av = *reinterpret_cast<const f32x4*>(a + lane * 16);
  const f32x4 bv = *reinterpret_cast<const f32x4*>(b + lane * 16);
#pragma unroll
  for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[j], bv[j], acc, 0, 0, 0);
}

// Byte offset of element (row, k) inside an A/B fragment.
template <class T>
__device__ __forceinline__ int frag_off(int row, int k);
template <>
__device__ __forceinline__ int frag_off<BF16>(int row, int k) {
  return (((k >> 3) * 32 + row) * 8 + (k & 7)) * 2;
}
template <>
__device__ __forceinline__ int frag_off<F32>(int row, int k) {
  // channel k of an 8-wide K step: lane half k/4, slot k%4.  MFMA j of the
  // four 32x32x2 steps pairs channels j and 4+j in A and B alike, so the K
  // order is a permutation shared by both operands and the sum is exact.
  return (((k >> 2) * 32 + row) * 4 + (k & 3)) * 4;
}

// ------------------------------------------------------- compile-time plan
__host__ __device__ constexpr int cmin(int a, int b) { return a < b ? a : b; }

template <int L, int M, bool GATE, int NW, int RT>
struct Plan {
  static constexpr int TE = 32 * RT;  // edges per workgroup
  // MFMA tiles per row tile for output degree l: G0 [+ gate] + (+/-) per m.
  static constexpr int ntype(int l) { return 1 + ((GATE && l >= 1) ? 1 : 0) + 2 * cmin(M, l); }
  // kept rows of degree l (row types): m = 0, then (+m, -m) for m <= min(M, l)
  static constexpr int nq(int l) { return 1 + 2 * cmin(M, l); }
  static constexpr int doff(int l) {
    int s = 0;
    for (int k = 0; k < l; ++k) s += nq(k) * (2 * k + 1);
    return s;
  }
  static constexpr int DS = doff(L + 1);  // kept Wigner entries per edge
  static constexpr int DP = (L + 1) + [] {  // kept rows per edge (d')
    int s = 0;
    for (int m = 1; m <= M; ++m) s += 2 * (L - m + 1);
    return s;
  }();
  // m-major position of row type q (0, +1, -1, +2, ...) of degree l
  static constexpr int mrow(int q, int l) {
    if (q == 0) return l;
    const int m = (q + 1) / 2;
    int base = L + 1;
    for (int k = 1; k < m; ++k) base += 2 * (L - k + 1);
    return base + ((q & 1) ? 0 : (L - m + 1)) + (l - m);
  }
  // B fragments per K step at input degree l.
  static constexpr int nbfrag(int l) {
    int s = (L + 1) + (GATE ? L : 0);
    for (int m = 1; m <= cmin(M, l); ++m) s += 4 * (L - m + 1);
    return s;
  }
  static constexpr int gbase(int m) {  // first B fragment of group m (m >= 1)
    int s = (L + 1) + (GATE ? L : 0);
    for (int k = 1; k < m; ++k) s += 4 * (L - k + 1);
    return s;
  }
  struct Tab {
    int owner[L + 1];
    int base[L + 1];
    int nslots[NW];
  };
  static constexpr Tab make() {
    Tab t{};
    int load[NW] = {};
    bool done[L + 1] = {};
    for (int it = 0; it <= L; ++it) {
      int best = -1;
      for (int l = L; l >= 0; --l)
        if (!done[l] && (best < 0 || ntype(l) > ntype(best))) best = l;
      int w = 0;
      for (int k = 1; k < NW; ++k)
        if (load[k] < load[w]) w = k;
      t.owner[best] = w;
      t.base[best] = load[w];
      load[w] += RT * ntype(best);
      done[best] = true;
    }
    for (int k = 0; k < NW; ++k) t.nslots[k] = load[k];
    return t;
  }
  static constexpr Tab tab = make();
  static constexpr int max_slots() {
    int m = 0;
    for (int k = 0; k < NW; ++k) m = tab.nslots[k] > m ? tab.nslots[k] : m;
    return m;
  }
  static constexpr int MS = max_slots();
  static constexpr int NT = NW * 64;
};

// Kept Wigner rows of one edge in the pair-major layout shared by the prep
// kernel, the dk workspace and the GEMM epilogue: per degree l, (l+1) column
// pairs (j = 2p, 2p+1; column 2l+1 is zero); each pair is a [q][2] block of
// the nq(l) kept row types, padded with zeros to a multiple of 4 floats, so
// one 16-byte read gives D(q, j) and D(q, j+1) of two row types.
template <int L, int M>
struct PairLayout {
  static constexpr int nq(int l) { return 1 + 2 * cmin(M, l); }
  static constexpr int pblk(int l) { return (2 * nq(l) + 3) / 4 * 4; }
  static constexpr int woff(int l) {
    int s = 0;
    for (int k = 0; k < l; ++k) s += (k + 1) * pblk(k);
    return s;
  }
  static constexpr int WS = woff(L + 1);  // floats per edge (a multiple of 4)
  // position of D(q, j) of degree l
  static constexpr int at(int l, int q, int j) { return woff(l) + (j >> 1) * pblk(l) + 2 * q + (j & 1); }
};

// FWD_EDGE: the forward GEMM whose gated output rows stay in the edge frame
// (Args::zout) for a second SO(2) convolution, instead of being rotated back
// and summed per node.  BWD_EDGE: the transposed GEMM of that second
// convolution with its output rows kept in the edge frame and passed through
// the gate backward (the gradient at the first convolution's output).
enum Mode { FWD = 0, BWD_DX = 1, FWD_EDGE = 2, BWD_EDGE = 3 };

struct Args {
  const void* a_src;      // [E_all, d', C_k] (TM raw): rotated rows, m-major, by edge id
  const float* dk;        // [E_all, WS] kept Wigner rows per edge id (pair layout)
  const int32_t* seg;     // [E] segment id per edge, non-decreasing
  const int32_t* eidx;    // [E] nullable: edge id of each kernel-order edge
  const void* rad;        // BWD_DX: [E_all, KR] (TM raw) or null
  void* drad;             // BWD_DX: [E_all, KR] (TM raw) output, nullable
  const void* rsave;      // BWD_DX: unscaled rotated forward inputs [E_all, d', C_n] (TM raw)
  const char* wpack;      // packed B fragments
  const float* bias;      // FWD: [N0] or null
  const float* jd;        // packed J_0..J_L
  float* out;             // [N_out, d, C_n]
  float* part;            // [ntiles, 2, d, C_n]
  int64_t E;
  int C_k, C_n;           // kernel input / output channels
  int n_cb;               // C_n / CB
  int extra;              // FWD: leading gate columns of W0 (= L * C_n if gated)
  int64_t ntiles;
  int64_t frags_per_cb;   // packed fragments per output-channel block
  void* gsave;            // FWD gated: [E_all, d' + L, C_n] (TM raw) pre-activation rows and
                          // gate rows, nullable; BWD_DX gated: a_src has d' + L rows
  void* zout;             // FWD_EDGE: [E_all, d', C_n] (TM raw) output rows (m-major), written
                          // in place of the inverse rotation and segment sum; BWD_EDGE:
                          // [E_all, d' + L, C_n], the gate backward of those rows at the
                          // pre-activations in gsave ([E_all, d' + L, C_n])
  int cb0;                // first output channel block (the grid covers n_cb blocks from it)
  int ow;                 // channels per row of out / part (0: C_n); output channel block cb
                          // lands at channel (cb - cb0) CB of its row when ow != 0
};

template <int L, int M>
__host__ __device__ constexpr int rad_slot(int q, int l, int c, int C) {
  // q: row type; m = (q + 1) / 2; slot = sum_{m' < m} (L - m' + 1) C + (l - m) C + c
  const int m = (q + 1) >> 1;
  int off = 0;
  for (int k = 0; k < m; ++k) off += (L - k + 1) * C;
  return off + (l - m) * C + c;
}


template <int L, int M>
__device__ __forceinline__ int rad_width(int C) {
  int w = 0;
  for (int m = 0; m <= M; ++m) w += (L - m + 1) * C;
  return w;
}

template <class F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
  (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}



// --------------------------------------------------------------- edge prep
// Per edge, once: the kept rows |m| <= mmax of its Wigner-D (from the Euler
// triple) and the rotated, optionally radially scaled operand of the SO(2)
// GEMM,  Y[e, (m, l), c] = sum_j D_l[e][(m), j] x[g(e), l^2 + j, c] (* rad),
// stored m-major by edge id ([E, d', C]), which is also the saved input of
// the weight gradient.  Replaces the bmm(wigner) + einsum(to_m) of
// esen_block.py:181,184 (and, with x = dL/dout gathered by dst, the rotation
// of the output gradient in the backward).
struct PrepArgs {
  const void* x;        // [N, d, C] (TX raw)
  const int32_t* gidx;  // [E] gather row per kernel-order edge
  const int32_t* eidx;  // [E] nullable: edge id per kernel-order edge
  const float* eulers;  // [E_all, 3] by edge id
  const void* rad;      // [E_all, KR] (TM raw) or null
  const float* jd;      // packed J_0..J_L
  void* y;              // [E_all, d', C] (TM raw) by edge id
  void* r;              // nullable: unscaled rows, same layout
  float* dk;            // [E_all, WS] kept Wigner rows by edge id (pair layout)
  int build_d;          // 1: compute and write dk; 0: read dk
  int64_t E;
  int C;
  const void* gsave;    // gated input gradient: the forward's pre-activation rows
                        // [E_all, d' + L, C] (TM raw); y then gets d' + L rows per edge:
                        // dL/dpre of the kept rows, then dL/dgate of degrees 1..L
  const int32_t* gidx2; // nullable: second gather row per edge (concatenated message
                        // [x[gidx] | x[gidx2] | x3[gidx3]]: channels [x_c, 2 x_c) from
                        // x[gidx2], [2 x_c, 3 x_c) from x3[gidx3])
  const void* x3;       // nullable: third source [*, d, x_c] (TX raw), per-edge rows
  const int32_t* gidx3; // its row per edge
  int x_c;              // channels of an x row (0: C)
};

template <class TX, int V>
__device__ __forceinline__ void load_vec(const typename TX::raw* p, float (&o)[V]);
template <>
__device__ __forceinline__ void load_vec<BF16, 8>(const uint16_t* p, float (&o)[8]) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    o[2 * k] = __uint_as_float(w[k] << 16);
    o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load_vec<F32, 8>(const float* p, float (&o)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p), b = *reinterpret_cast<const float4*>(p + 4);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
template <>
__device__ __forceinline__ void load_vec<BF16, 4>(const uint16_t* p, float (&o)[4]) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  o[0] = __uint_as_float(v.x << 16);
  o[1] = __uint_as_float(v.x & 0xffff0000u);
  o[2] = __uint_as_float(v.y << 16);
  o[3] = __uint_as_float(v.y & 0xffff0000u);
}
template <>
__device__ __forceinline__ void load_vec<F32, 4>(const float* p, float (&o)[4]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
}

// V elements (16 bytes of TM raw) already in registers -> fp32.
template <class TM, int V>
__device__ __forceinline__ void unpack_vec(uint4 v, float (&o)[V]);
template <>
__device__ __forceinline__ void unpack_vec<BF16, 8>(uint4 v, float (&o)[8]) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    o[2 * k] = __uint_as_float(w[k] << 16);
    o[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void unpack_vec<F32, 4>(uint4 v, float (&o)[4]) {
  o[0] = __uint_as_float(v.x); o[1] = __uint_as_float(v.y); o[2] = __uint_as_float(v.z); o[3] = __uint_as_float(v.w);
}

template <class TM, int V>
__device__ __forceinline__ void store_vec(typename TM::raw* p, const float (&v)[V]);
template <>
__device__ __forceinline__ void store_vec<BF16, 8>(uint16_t* p, const float (&v)[8]) {
  uint4 w;
  w.x = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  w.y = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
  w.z = f32_to_bf16(v[4]) | (static_cast<uint32_t>(f32_to_bf16(v[5])) << 16);
  w.w = f32_to_bf16(v[6]) | (static_cast<uint32_t>(f32_to_bf16(v[7])) << 16);
  *reinterpret_cast<uint4*>(p) = w;
}
template <>
__device__ __forceinline__ void store_vec<F32, 8>(float* p, const float (&v)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
template <>
__device__ __forceinline__ void store_vec<F32, 4>(float* p, const float (&v)[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store_vec<BF16, 4>(uint16_t* p, const float (&v)[4]) {
  uint2 w;
  w.x = f32_to_bf16(v[0]) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
  w.y = f32_to_bf16(v[2]) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}

// V elements of TM raw as one register vector (16 bytes, or 8 for 4 bf16).
template <class TM, int V>
struct RawVec {
  using type = uint4;
  static __device__ __forceinline__ void unpack(type v, float (&o)[V]) { unpack_vec<TM, V>(v, o); }
};
template <>
struct RawVec<BF16, 4> {
  using type = uint2;
  static __device__ __forceinline__ void unpack(uint2 v, float (&o)[4]) {
    o[0] = __uint_as_float(v.x << 16);
    o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16);
    o[3] = __uint_as_float(v.y & 0xffff0000u);
  }
};

// Edges and threads per prep workgroup (the grid is ceil(E / PREP_TE)).
constexpr int PREP_TE = 16;
constexpr int PREP_NT = 256;

template <int L, int M, class TM, class TX, bool GATED = false>
struct Prep {
  static constexpr int TE = PREP_TE;
  static constexpr int NT = PREP_NT;
  using P = Plan<L, M, false, 4, 1>;
  using PL = PairLayout<L, M>;
  static constexpr int WS = PL::WS;
  static constexpr int d = (L + 1) * (L + 1);
  // channels per item: 4 (16 bytes of fp32, 8 of bf16).  Eight bf16 channels
  // per item spilled at lmax > 4 or mmax > 2 and ran 12 % slower at lmax 4
  // (fewer resident waves).
  static constexpr int V = std::is_same_v<TM, BF16> ? 4 : TM::VEC;
  using RV = RawVec<TM, V>;

  struct Smem {
    float J[jd_size(L)];
    alignas(16) float D[TE * WS];
    float eul[TE * 3];
    int gid[TE];
    int gid2[TE];
    int gid3[TE];
    int eid[TE];
    float m2[TE * (2 * L + 1) * (2 * L + 1)];
    float trig[TE * 3 * 2 * (L + 1)];
  };

  static __device__ void build_d(Smem& s, int tid) {
    for (int q = tid; q < TE * 3 * (L + 1); q += NT) {
      const int e = q / (3 * (L + 1)), r = q % (3 * (L + 1));
      const int ang = r / (L + 1), m = r % (L + 1);
      float sn, cs;
      sincos_m(m, s.eul[e * 3 + ang], &sn, &cs);
      s.trig[(e * 3 + ang) * 2 * (L + 1) + m] = cs;
      s.trig[(e * 3 + ang) * 2 * (L + 1) + (L + 1) + m] = sn;
    }
    __syncthreads();
    for (int l = 0; l <= L; ++l) {
      const int n = 2 * l + 1;
      const float* J = s.J + jd_offset(l);
      for (int q = tid; q < TE * n; q += NT) {
        const int e = q / n, k = q % n;
        const float* tb = s.trig + (e * 3 + 1) * 2 * (L + 1);
        const float* tc = s.trig + (e * 3 + 2) * 2 * (L + 1);
        wigner_m2_row(l, k, J, tb, tb + (L + 1), tc, tc + (L + 1), s.m2 + (e * n + k) * n);
      }
      __syncthreads();
      const int nql = P::nq(l);
      for (int q = tid; q < TE * nql * n; q += NT) {
        const int e = q / (nql * n), r = q % (nql * n);
        const int qi = r / n, j = r % n;
        const int mm = (qi + 1) >> 1;
        const int i = (qi == 0) ? l : ((qi & 1) ? l + mm : l - mm);
        const int ii = 2 * l - i;
        const float* ta = s.trig + (e * 3 + 0) * 2 * (L + 1);
        const float* M2 = s.m2 + e * n * n;
        float va = 0.f, vb = 0.f;
        for (int k = 0; k < n; ++k) {
          va = fmaf(J[i * n + k], M2[k * n + j], va);
          vb = fmaf(J[ii * n + k], M2[k * n + j], vb);
        }
        float v = va;
        if (i != l) {
          const int f = l - i;
          v = xcos(ta, f) * va + xsin(ta + (L + 1), f) * vb;
        }
        s.D[e * WS + PL::woff(l) + (j >> 1) * PL::pblk(l) + 2 * qi + (j & 1)] = v;
      }
      __syncthreads();
    }
  }

  // Gated input gradient (GateActivation backward, activation.py:57-77): with
  // o the rotated output gradient and z the saved pre-activations,
  //   l = 0:  dpre = o SiLU'(z) = o s (1 + z (1 - s)),  s = sigmoid(z);
  //   l >= 1: t = tanh(z_gate[l]); dpre_q = o_q t;  dgate[l] = (1 - t^2) sum_q o_q z_q.
  static __device__ void run_gated_bwd(const Smem& s, const PrepArgs& a, int nvalid, int tid) {
    constexpr int DG = P::DP + L;  // rows per edge of the saved and written arrays
    const int nch = a.C / V;
    for (int u = tid; u < nvalid * nch; u += NT) {
      const int e = u / nch, c0 = (u - e * nch) * V;
      const int64_t eid = s.eid[e];
      const typename TX::raw* xg = reinterpret_cast<const typename TX::raw*>(a.x) +
                                   static_cast<int64_t>(s.gid[e]) * d * a.C + c0;
      typename TM::raw* yo = reinterpret_cast<typename TM::raw*>(a.y) + eid * DG * a.C + c0;
      const typename TM::raw* zs = reinterpret_cast<const typename TM::raw*>(a.gsave) + eid * DG * a.C + c0;
      static_for<L + 1>([&](auto LI) {
        constexpr int l = decltype(LI)::value;
        constexpr int n = 2 * l + 1;
        float xv[n][V];
#pragma unroll
        for (int j = 0; j < n; ++j) load_vec<TX, V>(xg + (l * l + j) * a.C, xv[j]);
        const float* Dl = s.D + e * WS;
        float o[P::nq(l)][V];
#pragma unroll
        for (int q = 0; q < P::nq(l); ++q)
#pragma unroll
          for (int c = 0; c < V; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < n; ++j) acc = fmaf(Dl[PL::at(l, q, j)], xv[j][c], acc);
            o[q][c] = acc;
          }
        if constexpr (l == 0) {
          float z[V];
          load_vec<TM, V>(zs + static_cast<int64_t>(P::mrow(0, 0)) * a.C, z);
#pragma unroll
          for (int c = 0; c < V; ++c) {
            const float sg = 1.0f / (1.0f + expf(-z[c]));
            o[0][c] *= sg * (1.0f + z[c] * (1.0f - sg));
          }
          store_vec<TM, V>(yo + static_cast<int64_t>(P::mrow(0, 0)) * a.C, o[0]);
        } else {
          float t[V], dg[V];
          load_vec<TM, V>(zs + static_cast<int64_t>(P::DP + l - 1) * a.C, t);
#pragma unroll
          for (int c = 0; c < V; ++c) {
            t[c] = tanhf(t[c]);
            dg[c] = 0.f;
          }
#pragma unroll
          for (int q = 0; q < P::nq(l); ++q) {
            float z[V];
            load_vec<TM, V>(zs + static_cast<int64_t>(P::mrow(q, l)) * a.C, z);
#pragma unroll
            for (int c = 0; c < V; ++c) {
              dg[c] = fmaf(o[q][c], z[c], dg[c]);
              o[q][c] *= t[c];
            }
            store_vec<TM, V>(yo + static_cast<int64_t>(P::mrow(q, l)) * a.C, o[q]);
          }
#pragma unroll
          for (int c = 0; c < V; ++c) dg[c] *= (1.0f - t[c] * t[c]);
          store_vec<TM, V>(yo + static_cast<int64_t>(P::DP + l - 1) * a.C, dg);
        }
      });
    }
  }

  static __device__ void run(const PrepArgs& a) {
    __shared__ Smem s;
    const int tid = threadIdx.x;
    const int64_t e0 = static_cast<int64_t>(blockIdx.x) * TE;
    const int nvalid = static_cast<int>((a.E - e0) < TE ? (a.E - e0) : TE);
    for (int i = tid; i < jd_size(L); i += NT) s.J[i] = a.jd[i];
    if (tid < TE) {
      const bool v = tid < nvalid;
      const int64_t p = e0 + tid;
      const int ei = v ? (a.eidx ? a.eidx[p] : static_cast<int>(p)) : -1;
      s.eid[tid] = ei;
      s.gid[tid] = v ? a.gidx[p] : 0;
      s.gid2[tid] = (v && a.gidx2) ? a.gidx2[p] : 0;
      s.gid3[tid] = (v && a.gidx3) ? a.gidx3[p] : 0;
      for (int k = 0; k < 3; ++k)
        s.eul[tid * 3 + k] = (v && a.build_d) ? a.eulers[static_cast<int64_t>(ei) * 3 + k] : 0.f;
    }
    __syncthreads();
    if (a.build_d) {
      // pads of the pair layout stay zero
      for (int i = tid; i < TE * WS; i += NT) s.D[i] = 0.f;
      __syncthreads();
      build_d(s, tid);
      float4* dk4 = reinterpret_cast<float4*>(a.dk);
      const float4* d4 = reinterpret_cast<const float4*>(s.D);
      for (int i = tid; i < nvalid * (WS / 4); i += NT) {
        const int e = i / (WS / 4), k = i - e * (WS / 4);
        dk4[static_cast<int64_t>(s.eid[e]) * (WS / 4) + k] = d4[i];
      }
    } else {
      const float4* dk4 = reinterpret_cast<const float4*>(a.dk);
      float4* d4 = reinterpret_cast<float4*>(s.D);
      for (int i = tid; i < TE * (WS / 4); i += NT) {
        const int e = i / (WS / 4), k = i - e * (WS / 4);
        d4[i] = s.eid[e] >= 0 ? dk4[static_cast<int64_t>(s.eid[e]) * (WS / 4) + k] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      __syncthreads();
    }
    const int nch = a.C / V;
    const int64_t rw = rad_width<L, M>(a.C);
    if constexpr (GATED) {  // its own instantiation: the common path keeps its register budget
      run_gated_bwd(s, a, nvalid, tid);
      return;
    }
    // concatenated message: channels [0, xc) from x[gidx], [xc, 2 xc) from
    // x[gidx2], [2 xc, 3 xc) from x3[gidx3]
    const int xc = a.x_c > 0 ? a.x_c : a.C;
    for (int u = tid; u < nvalid * nch; u += NT) {
      const int e = u / nch, c0 = (u - e * nch) * V;
      const int64_t eid = s.eid[e];
      const int part = (c0 >= xc) + (c0 >= 2 * xc);
      const int g = part == 0 ? s.gid[e] : (part == 1 ? s.gid2[e] : s.gid3[e]);
      const typename TX::raw* xg = reinterpret_cast<const typename TX::raw*>(part == 2 ? a.x3 : a.x) +
                                   static_cast<int64_t>(g) * d * xc + (c0 - part * xc);
      typename TM::raw* yo = reinterpret_cast<typename TM::raw*>(a.y) + eid * P::DP * a.C + c0;
      typename TM::raw* ro = a.r ? reinterpret_cast<typename TM::raw*>(a.r) + eid * P::DP * a.C + c0 : nullptr;
      const typename TM::raw* rp = a.rad ? reinterpret_cast<const typename TM::raw*>(a.rad) + eid * rw + c0 : nullptr;
      // all radial slots of this (edge, channel chunk) in flight at once: one
      // memory latency per item instead of one per kept row.  Where holding
      // them all beside the largest degree's x rows would not fit the register
      // budget (and spilled: bf16 at lmax 6, mmax = lmax), each degree loads
      // its own min(mmax, l) + 1 slots with its x rows instead.
      constexpr int NSLOT = rad_slot<L, M>(2 * M, L, 0, 1) + 1;  // sum_m (L - m + 1)
      constexpr bool ALL = NSLOT * 4 + (2 * L + 1) * V <= 120;
      typename RV::type rr[ALL ? NSLOT : 1];
      if (ALL && rp) {
#pragma unroll
        for (int k = 0; k < NSLOT; ++k)
          rr[k] = *reinterpret_cast<const typename RV::type*>(rp + static_cast<int64_t>(k) * a.C);
      }
      static_for<L + 1>([&](auto LI) {
        constexpr int l = decltype(LI)::value;
        constexpr int n = 2 * l + 1;
        constexpr int NM = cmin(M, l) + 1;
        typename RV::type rl[ALL ? 1 : NM];  // this degree's slots, by m
        if (!ALL && rp) {
#pragma unroll
          for (int m = 0; m < (ALL ? 1 : NM); ++m)
            rl[m] = *reinterpret_cast<const typename RV::type*>(
                rp + static_cast<int64_t>(rad_slot<L, M>(2 * m, l, 0, 1)) * a.C);
        }
        float xv[n][V];
#pragma unroll
        for (int j = 0; j < n; ++j) load_vec<TX, V>(xg + (l * l + j) * xc, xv[j]);
        const float* Dl = s.D + e * WS;
#pragma unroll
        for (int q = 0; q < P::nq(l); ++q) {
          float o[V];
#pragma unroll
          for (int c = 0; c < V; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < n; ++j) acc = fmaf(Dl[PL::at(l, q, j)], xv[j][c], acc);
            o[c] = acc;
          }
          const int64_t ro_off = static_cast<int64_t>(P::mrow(q, l)) * a.C;
          if (ro) store_vec<TM, V>(ro + ro_off, o);
          if (rp) {
            float rv[V];
            if constexpr (ALL)
              RV::unpack(rr[rad_slot<L, M>(q, l, 0, 1)], rv);
            else
              RV::unpack(rl[(q + 1) >> 1], rv);
#pragma unroll
            for (int c = 0; c < V; ++c) o[c] *= rv[c];
          }
          store_vec<TM, V>(yo + ro_off, o);
        }
      });
    }
  }
};

// Three resident workgroups per CU (at most 170 registers): the compiler then
// keeps the Wigner coefficients of degree 6 at mmax 6 in LDS instead of
// holding all 169 of them in registers (212 -> 167 VGPRs, no spills); the
// other shapes already fit.  The gated backward would spill under it.
template <int L, int M, class TM, class TX, bool GATED = false>
__global__ __launch_bounds__(PREP_NT, GATED ? 1 : 3) void prep_kernel(PrepArgs a) {
  Prep<L, M, TM, TX, GATED>::run(a);
}

}  // namespace msg
}  // namespace maloq
