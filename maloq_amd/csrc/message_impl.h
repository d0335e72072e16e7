#pragma once
// Device code of the fused equivariant message block on gfx950:
//   gather x[src] -> rotate into the edge frame (kept rows |m| <= mmax of D)
//   -> [radial scale] -> SO(2) per-m linear on MFMA (bf16 or fp32 operands,
//   fp32 accumulation) [+ bias, gate] -> inverse rotation -> sorted-segment
//   sum into nodes.
//
// Replaces Edgewise.forward_node (helm/esen_block.py:146-208): the dense
// bmm(wigner), einsum(to_m), SO2_Convolution (helm/nn/so2_layers.py:139-214),
// GateActivation (helm/nn/activation.py:57-77), einsum(to_m^T),
// bmm(wigner_inv) and index_add_ all happen in one kernel, so edge features
// never round-trip through HBM.  The same kernel, with transposed packed
// weights and the radial scale moved to the epilogue, computes the input
// gradient of the block (edges ordered by source there).
//
// Tiling.  A workgroup owns TE = 32 * RT consecutive edges (sorted by segment id)
// and CB = 32 output channels.  The SO(2) linear is written as three (or more)
// real GEMMs, one per |m|: for m > 0 the +m / -m rows are stacked along K and
// the complex mix is folded into a packed [[Wr, Wi], [-Wi, Wr]] weight, so
// every MFMA is a plain real product.  The K loop runs over (l_in, 16 or 8
// input channels); per step the rotated A fragments (one per kept row type and
// 32-edge row tile) and the packed B fragments live in LDS in the exact lane
// order of v_mfma_f32_32x32x16_bf16 / v_mfma_f32_32x32x2f32 (1 KB per
// fragment, one 16-byte ds_read per lane).  Each wave owns whole output
// degrees l_out (all row tiles and all |m| tiles of that l_out), assigned by
// a compile-time longest-processing-time schedule, so the inverse rotation is
// done in registers straight from the accumulators and the segment sum stays
// wave-local.  Segments cut by a tile boundary are written to a partials
// buffer and summed in tile order by message_fixup_kernel (deterministic).
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
  // LDS layout (bytes)
  static constexpr int A_BYTES = (2 * M + 1) * RT * FRAG;
  static constexpr int B_BYTES = nbfrag(L) * FRAG;
  static constexpr int M2_BYTES = TE * (2 * L + 1) * (2 * L + 1) * 4 + TE * 3 * 2 * (L + 1) * 4;
  static constexpr int EPI_BYTES = NW * TE * 33 * 4;
  static constexpr int cmax(int a, int b) { return a > b ? a : b; }
  static constexpr int STAGE_BYTES = cmax(A_BYTES + B_BYTES, EPI_BYTES);
};

enum Mode { FWD = 0, BWD_DX = 1 };

struct Args {
  const void* a_src;      // [E_all, d', C_k] (TM raw): rotated rows, m-major, by edge id
  const float* dk;        // [E_all, DS] kept Wigner rows per edge id
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
};

template <int L, int M>
__device__ __forceinline__ int rad_slot(int q, int l, int c, int C) {
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

// ------------------------------------------------------------------ kernel
template <int L, int M, bool GATE, int NW, int RT, class TM, class TX, int MODE>
struct Kernel {
  using P = Plan<L, M, GATE, NW, RT>;
  static constexpr int TE = P::TE;
  static constexpr int d = (L + 1) * (L + 1);
  static constexpr int NT = P::NT;
  static constexpr int KC = TM::KC;

  struct Smem {
    float D[TE * P::DS];
    int seg[TE];
    int eid[TE];
    alignas(16) char stage[P::STAGE_BYTES];
  };

  // ------------------------------------------------------------ prologue
  // A fragments of one K step: for every kept row type q of degree LI and
  // 32-edge row tile rt, lane (row, half) copies 16 bytes of the rotated rows
  // (channels c0 + half * VEC ...) straight into fragment order.
  template <int LI>
  static __device__ __forceinline__ void stage_a(Smem& s, const Args& a, int wave, int lane,
                                                 int c0) {
    constexpr int nql = P::nq(LI);
    const int row = lane & 31, half = lane >> 5;
    for (int f = wave; f < nql * RT; f += NW) {
      const int q = f / RT, rt = f % RT;
      const int e = rt * 32 + row;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      if (s.eid[e] >= 0) {
        const typename TM::raw* src = reinterpret_cast<const typename TM::raw*>(a.a_src) +
                                      (static_cast<int64_t>(s.eid[e]) * P::DP + P::mrow(q, LI)) * a.C_k +
                                      c0 + half * TM::VEC;
        v = *reinterpret_cast<const uint4*>(src);
      }
      *reinterpret_cast<uint4*>(s.stage + (q * RT + rt) * FRAG + lane * 16) = v;
    }
  }

  static __device__ __forceinline__ void stage_b(Smem& s, const char* src, int nfrag, int tid) {
    const uint4* g = reinterpret_cast<const uint4*>(src);
    uint4* d4 = reinterpret_cast<uint4*>(s.stage + P::A_BYTES);
    const int n16 = nfrag * (FRAG / 16);
    for (int i = tid; i < n16; i += NT) d4[i] = g[i];
  }

  // ------------------------------------------------------------ MFMA step
  // slot of (degree l, row tile rt, tile type t); t: 0 = G0, [1 = gate],
  // then (+,-) pairs per m.
  template <int l, int rt>
  static constexpr int slot0() { return P::tab.base[l] + rt * P::ntype(l); }
  template <int l>
  static constexpr int gt() { return (GATE && l >= 1) ? 1 : 0; }

  template <int W, int LI>
  static __device__ __forceinline__ void mma_step(f32x16 (&acc)[P::MS], const Smem& s, int lane) {
    const char* A = s.stage;
    const char* B = s.stage + P::A_BYTES;
    static_for<L + 1>([&](auto LO) {
      constexpr int l = decltype(LO)::value;
      if constexpr (P::tab.owner[l] == W) {
        static_for<RT>([&](auto RTI) {
          constexpr int rt = decltype(RTI)::value;
          constexpr int sb = slot0<l, rt>();
          const char* A0 = A + (0 * RT + rt) * FRAG;
          mma(acc[sb], A0, B + l * FRAG, lane, TM{});
          if constexpr (GATE && l >= 1) mma(acc[sb + 1], A0, B + (L + 1 + (l - 1)) * FRAG, lane, TM{});
          static_for<M>([&](auto MI) {
            constexpr int m = decltype(MI)::value + 1;
            if constexpr (m <= l && m <= LI) {
              const char* Ap = A + ((2 * m - 1) * RT + rt) * FRAG;
              const char* Am = A + ((2 * m) * RT + rt) * FRAG;
              constexpr int gb = P::gbase(m), nl = L - m + 1, lo = l - m;
              static_for<2>([&](auto PMI) {
                constexpr int pm = decltype(PMI)::value;
                constexpr int sl = sb + gt<l>() + 1 + 2 * (m - 1) + pm;
                mma(acc[sl], Ap, B + (gb + (0 * 2 + pm) * nl + lo) * FRAG, lane, TM{});
                mma(acc[sl], Am, B + (gb + (1 * 2 + pm) * nl + lo) * FRAG, lane, TM{});
              });
            }
          });
        });
      }
    });
  }

  template <int LI>
  static __device__ __forceinline__ void mma_dispatch(f32x16 (&acc)[P::MS], const Smem& s,
                                                      int wave, int lane) {
    static_for<NW>([&](auto WI) {
      constexpr int w = decltype(WI)::value;
      if (wave == w) mma_step<w, LI>(acc, s, lane);
    });
  }

  template <int LI>
  static __device__ void kloop(f32x16 (&acc)[P::MS], Smem& s, const Args& a, int cb, int tid,
                               int wave, int lane) {
    const int nks = a.C_k / KC;
    int64_t foff = 0;
    for (int l = 0; l < LI; ++l) foff += static_cast<int64_t>(P::nbfrag(l)) * nks;
    const char* wbase = a.wpack + (static_cast<int64_t>(cb) * a.frags_per_cb + foff) * FRAG;
    constexpr int nb = P::nbfrag(LI);
    for (int ks = 0; ks < nks; ++ks) {
      stage_a<LI>(s, a, wave, lane, ks * KC);
      stage_b(s, wbase + static_cast<int64_t>(ks) * nb * FRAG, nb, tid);
      __syncthreads();
      mma_dispatch<LI>(acc, s, wave, lane);
      __syncthreads();
    }
  }

  // ------------------------------------------------------------ epilogue
  template <int W, int l>
  static __device__ void epi_degree(f32x16 (&acc)[P::MS], Smem& s, const Args& a, int64_t tile,
                                    int cb, int wave, int lane, int nvalid, bool first_partial,
                                    bool last_partial) {
    constexpr int n = 2 * l + 1;
    float* stage = reinterpret_cast<float*>(s.stage) + wave * TE * 33;
    const int co = lane & 31;
    const int col = cb * CB + co;
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      constexpr int sb = slot0<l, rt>();
      if constexpr (MODE == FWD) {
        if (a.bias != nullptr) {
          const float b0 = a.bias[a.extra + l * a.C_n + col];
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[sb][i] += b0;
          if constexpr (GATE && l >= 1) {
            const float bg = a.bias[(l - 1) * a.C_n + col];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[sb + 1][i] += bg;
          }
        }
        if constexpr (GATE) {
          if constexpr (l == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float z = acc[sb][i];
              acc[sb][i] = z / (1.0f + __expf(-z));
            }
          } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const float g = tanhf(acc[sb + 1][i]);
              acc[sb][i] *= g;
              static_for<M>([&](auto MI) {
                constexpr int m = decltype(MI)::value + 1;
                if constexpr (m <= l) {
                  acc[sb + 2 + 2 * (m - 1)][i] *= g;
                  acc[sb + 3 + 2 * (m - 1)][i] *= g;
                }
              });
            }
          }
        }
      } else {
        bwd_radial<l, rt, sb>(acc, s, a, col, lane);
      }
    });
    for (int j = 0; j < n; ++j) {
      static_for<RT>([&](auto RTI) {
        constexpr int rt = decltype(RTI)::value;
        constexpr int sb = slot0<l, rt>();
        constexpr int g1 = gt<l>() + 1;
        static_for<16>([&](auto II) {
          constexpr int i = decltype(II)::value;
          const int e = rt * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
          const float* Dl = s.D + e * P::DS + P::doff(l);
          float v = Dl[j] * acc[sb][i];
          static_for<M>([&](auto MI) {
            constexpr int m = decltype(MI)::value + 1;
            if constexpr (m <= l) {
              v = fmaf(Dl[(2 * m - 1) * n + j], acc[sb + g1 + 2 * (m - 1)][i], v);
              v = fmaf(Dl[(2 * m) * n + j], acc[sb + g1 + 1 + 2 * (m - 1)][i], v);
            }
          });
          stage[e * 33 + co] = v;
        });
      });
      wave_sync();
      if (lane < 32) {
        float sum = 0.f;
        int cur = s.seg[0];
        bool first = true;
        const int64_t rowoff = static_cast<int64_t>(l * l + j) * a.C_n + col;
        for (int r = 0; r < nvalid; ++r) {
          sum += stage[r * 33 + co];
          const bool last = (r + 1 == nvalid);
          if (last || s.seg[r + 1] != cur) {
            if ((first && first_partial) || (last && last_partial)) {
              const int slot = first ? 0 : 1;
              a.part[(tile * 2 + slot) * d * a.C_n + rowoff] = sum;
            } else {
              a.out[static_cast<int64_t>(cur) * d * a.C_n + rowoff] = sum;
            }
            sum = 0.f;
            first = false;
            if (!last) cur = s.seg[r + 1];
          }
        }
      }
      wave_sync();
    }
  }

  // BWD_DX: the accumulators hold dY on the forward-input side of degree l.
  // Writes d(rad) = sum_(+/-) dY * R (R: unscaled rotated forward inputs, saved
  // by the forward) and scales dY by rad before the inverse rotation.
  template <int l, int rt, int sb>
  static __device__ __forceinline__ void bwd_radial(f32x16 (&acc)[P::MS], Smem& s, const Args& a,
                                                    int col, int lane) {
    if (a.rad == nullptr) return;
    const int64_t rw = rad_width<L, M>(a.C_n);
    static_for<16>([&](auto II) {
      constexpr int i = decltype(II)::value;
      const int e = rt * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
      if (s.eid[e] < 0) return;
      const int64_t eo = static_cast<int64_t>(s.eid[e]) * rw;
      const typename TM::raw* rp = reinterpret_cast<const typename TM::raw*>(a.rad) + eo;
      const typename TM::raw* rs = reinterpret_cast<const typename TM::raw*>(a.rsave) +
                                   static_cast<int64_t>(s.eid[e]) * P::DP * a.C_n + col;
      {
        const int slot = rad_slot<L, M>(0, l, col, a.C_n);
        const float dy = acc[sb][i];
        if (a.drad)
          reinterpret_cast<typename TM::raw*>(a.drad)[eo + slot] =
              TM::cvt(dy * TM::load(rs + P::mrow(0, l) * a.C_n));
        acc[sb][i] = dy * TM::load(rp + slot);
      }
      static_for<M>([&](auto MI) {
        constexpr int m = decltype(MI)::value + 1;
        if constexpr (m <= l) {
          const int slot = rad_slot<L, M>(2 * m - 1, l, col, a.C_n);
          const float r = TM::load(rp + slot);
          const float dyp = acc[sb + 1 + 2 * (m - 1)][i], dym = acc[sb + 2 + 2 * (m - 1)][i];
          if (a.drad)
            reinterpret_cast<typename TM::raw*>(a.drad)[eo + slot] =
                TM::cvt(dyp * TM::load(rs + P::mrow(2 * m - 1, l) * a.C_n) +
                        dym * TM::load(rs + P::mrow(2 * m, l) * a.C_n));
          acc[sb + 1 + 2 * (m - 1)][i] = dyp * r;
          acc[sb + 2 + 2 * (m - 1)][i] = dym * r;
        }
      });
    });
  }

  template <int W>
  static __device__ void epilogue(f32x16 (&acc)[P::MS], Smem& s, const Args& a, int64_t tile,
                                  int cb, int wave, int lane, int nvalid, bool fp, bool lp) {
    static_for<L + 1>([&](auto LO) {
      constexpr int l = decltype(LO)::value;
      if constexpr (P::tab.owner[l] == W) epi_degree<W, l>(acc, s, a, tile, cb, wave, lane, nvalid, fp, lp);
    });
  }

  static __device__ void run(const Args& a) {
    __shared__ Smem s;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // XCD-aware mapping: workgroups of one channel block share a set of XCDs
    // (consecutive workgroup ids are dispatched round-robin over the 8 XCDs),
    // so each XCD's L2 holds the packed weights of fewer channel blocks.
    const int64_t bid = blockIdx.x;
    int64_t tile;
    int cb;
    if (a.n_cb > 1 && (8 % a.n_cb) == 0) {
      const int per = 8 / a.n_cb;
      const int xcd = static_cast<int>(bid % 8);
      cb = xcd / per;
      tile = (bid / 8) * per + (xcd % per);
    } else {
      cb = static_cast<int>(bid % a.n_cb);
      tile = bid / a.n_cb;
    }
    if (tile >= a.ntiles) return;  // whole workgroup exits together
    const int64_t e0 = tile * TE;
    const int nvalid = static_cast<int>((a.E - e0) < TE ? (a.E - e0) : TE);
    if (tid < TE) {
      const bool v = tid < nvalid;
      const int64_t p = e0 + tid;
      s.seg[tid] = v ? a.seg[p] : -1;
      s.eid[tid] = v ? (a.eidx ? a.eidx[p] : static_cast<int>(p)) : -1;
    }
    __syncthreads();
    // kept Wigner rows of the tile's edges
    for (int i = tid; i < TE * P::DS; i += NT) {
      const int e = i / P::DS, k = i - e * P::DS;
      s.D[i] = s.eid[e] >= 0 ? a.dk[static_cast<int64_t>(s.eid[e]) * P::DS + k] : 0.f;
    }
    __syncthreads();
    const bool first_partial = (e0 > 0) && (a.seg[e0 - 1] == a.seg[e0]);
    const bool last_partial =
        (e0 + nvalid < a.E) && (a.seg[e0 + nvalid] == a.seg[e0 + nvalid - 1]);
    f32x16 acc[P::MS];
#pragma unroll
    for (int k = 0; k < P::MS; ++k)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[k][i] = 0.f;

    static_for<L + 1>([&](auto LI) {
      kloop<decltype(LI)::value>(acc, s, a, cb, tid, wave, lane);
    });

    static_for<NW>([&](auto WI) {
      constexpr int w = decltype(WI)::value;
      if (wave == w) epilogue<w>(acc, s, a, tile, cb, wave, lane, nvalid, first_partial, last_partial);
    });
  }
};

template <int L, int M, bool GATE, int NW, int RT, class TM, class TX, int MODE>
__global__ __launch_bounds__(NW * 64, (NW == 4 ? 2 : 1)) void message_kernel(Args a) {
  Kernel<L, M, GATE, NW, RT, TM, TX, MODE>::run(a);
}

}  // namespace msg
}  // namespace maloq


namespace maloq {
namespace msg {

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
  float* dk;            // [E_all, DS] kept Wigner rows by edge id
  int build_d;          // 1: compute and write dk; 0: read dk
  int64_t E;
  int C;
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
__device__ __forceinline__ void load_vec<F32, 4>(const float* p, float (&o)[4]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
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
__device__ __forceinline__ void store_vec<F32, 4>(float* p, const float (&v)[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

template <int L, int M, class TM, class TX>
struct Prep {
  static constexpr int TE = 32;
  static constexpr int NT = 256;
  using P = Plan<L, M, false, 4, 1>;
  static constexpr int d = (L + 1) * (L + 1);
  static constexpr int V = TM::VEC;

  struct Smem {
    float J[jd_size(L)];
    float D[TE * P::DS];
    float eul[TE * 3];
    int gid[TE];
    int eid[TE];
    float m2[TE * (2 * L + 1) * (2 * L + 1)];
    float trig[TE * 3 * 2 * (L + 1)];
  };

  static __device__ void build_d(Smem& s, int tid) {
    for (int q = tid; q < TE * 3 * (L + 1); q += NT) {
      const int e = q / (3 * (L + 1)), r = q % (3 * (L + 1));
      const int ang = r / (L + 1), m = r % (L + 1);
      float sn, cs;
      sincosf(static_cast<float>(m) * s.eul[e * 3 + ang], &sn, &cs);
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
      const int dof = P::doff(l);
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
        s.D[e * P::DS + dof + qi * n + j] = v;
      }
      __syncthreads();
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
      for (int k = 0; k < 3; ++k)
        s.eul[tid * 3 + k] = (v && a.build_d) ? a.eulers[static_cast<int64_t>(ei) * 3 + k] : 0.f;
    }
    __syncthreads();
    if (a.build_d) {
      build_d(s, tid);
      for (int i = tid; i < nvalid * P::DS; i += NT) {
        const int e = i / P::DS, k = i - e * P::DS;
        a.dk[static_cast<int64_t>(s.eid[e]) * P::DS + k] = s.D[i];
      }
    } else {
      for (int i = tid; i < TE * P::DS; i += NT) {
        const int e = i / P::DS, k = i - e * P::DS;
        s.D[i] = s.eid[e] >= 0 ? a.dk[static_cast<int64_t>(s.eid[e]) * P::DS + k] : 0.f;
      }
      __syncthreads();
    }
    const int nch = a.C / V;
    const int64_t rw = rad_width<L, M>(a.C);
    for (int u = tid; u < nvalid * nch; u += NT) {
      const int e = u / nch, c0 = (u - e * nch) * V;
      const int64_t eid = s.eid[e];
      const typename TX::raw* xg = reinterpret_cast<const typename TX::raw*>(a.x) +
                                   static_cast<int64_t>(s.gid[e]) * d * a.C + c0;
      typename TM::raw* yo = reinterpret_cast<typename TM::raw*>(a.y) + eid * P::DP * a.C + c0;
      typename TM::raw* ro = a.r ? reinterpret_cast<typename TM::raw*>(a.r) + eid * P::DP * a.C + c0 : nullptr;
      const typename TM::raw* rp = a.rad ? reinterpret_cast<const typename TM::raw*>(a.rad) + eid * rw + c0 : nullptr;
      static_for<L + 1>([&](auto LI) {
        constexpr int l = decltype(LI)::value;
        constexpr int n = 2 * l + 1;
        float xv[n][V];
#pragma unroll
        for (int j = 0; j < n; ++j) load_vec<TX, V>(xg + (l * l + j) * a.C, xv[j]);
        const float* Dl = s.D + e * P::DS + P::doff(l);
#pragma unroll
        for (int q = 0; q < P::nq(l); ++q) {
          float o[V];
#pragma unroll
          for (int c = 0; c < V; ++c) {
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < n; ++j) acc = fmaf(Dl[q * n + j], xv[j][c], acc);
            o[c] = acc;
          }
          const int64_t ro_off = static_cast<int64_t>(P::mrow(q, l)) * a.C;
          if (ro) store_vec<TM, V>(ro + ro_off, o);
          if (rp) {
            float rv[V];
            load_vec<TM, V>(rp + rad_slot<L, M>(q, l, 0, a.C), rv);
#pragma unroll
            for (int c = 0; c < V; ++c) o[c] *= rv[c];
          }
          store_vec<TM, V>(yo + ro_off, o);
        }
      });
    }
  }
};

template <int L, int M, class TM, class TX>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a) {
  Prep<L, M, TM, TX>::run(a);
}

}  // namespace msg
}  // namespace maloq
