#pragma once
// The SO(2) GEMM of the fused message block with its inverse-rotation and
// sorted-segment-sum epilogue (gfx950, MFMA 32x32).
//
// Input rows: Y [E, d', C_k] (m-major kept rows of D x[src] (*) rad, written by
// the prep kernel) for the forward; the rotated output gradient for the input
// gradient (edges in source order, rows gathered through eidx).
//
// Work split.  A workgroup (NW waves) owns TE = 32 RT consecutive edges of the
// segment-sorted order and CB = 32 kernel-output channels.  Each wave owns a
// set of whole output degrees l_out (compile-time longest-processing-time
// schedule over the MFMA work of each degree) for all RT row tiles, so the
// inverse rotation runs from its own accumulators and the segment sum stays
// inside the wave.  The K loop runs over (l_in, KC input channels):
//   * A (rotated rows): one 1 KB fragment per (row type q of l_in, row tile),
//     in the exact lane order of the MFMA A operand; loaded from global into
//     registers one step ahead, stored to a double-buffered LDS stage, one
//     barrier per step.  Every wave reads the fragments it needs from LDS.
//   * B (weights): each wave loads only the fragments of its own degrees
//     straight from global memory into registers (16 bytes per lane, fully
//     coalesced; packed on the host in lane order), one step ahead.  For
//     m > 0 only Wr and Wi are stored; the complex mix
//         y+ = Wr x+ - Wi x-,  y- = Wi x+ + Wr x-        (so2_layers.py:61-67)
//     and its transpose (input gradient: dx+ = Wr^T dy+ + Wi^T dy-,
//     dx- = -Wi^T dy+ + Wr^T dy-) negate a register copy of Wi.
// Epilogue per owned degree l: [bias, gate | radial scale and its gradient],
// then for each pair of output columns (j, j+1) and each 16-edge chunk:
// v = sum_q D(q, j) acc_q per row (Wigner rows in LDS in a pair-major layout,
// one 16-byte read per (row, 2 j)), staged through LDS so that lane (c, h)
// holds column j + h of all 16 rows, then a running sum over the edges in
// order with uniform control (segment ends from a 64-bit ballot mask); each
// finished segment is stored once (or to the partials buffer when it is cut
// by a tile boundary).  Deterministic: fixed summation order, no atomics.
#include "message_impl.h"

namespace maloq {
namespace msg {

template <int L, int M, bool GATE, int NW, int RT>
struct GPlan {
  static constexpr int TE = 32 * RT;
  static constexpr int NT = NW * 64;
  static_assert(TE <= 64, "segment masks are 64-bit");
  static constexpr int gt(int l) { return (GATE && l >= 1) ? 1 : 0; }
  static constexpr int nq(int l) { return 1 + 2 * cmin(M, l); }
  static constexpr int ntype(int l) { return nq(l) + gt(l); }
  // accumulator type of row type q of degree l (0: m=0, [1: gate], then +1, -1, +2, ...)
  static constexpr int qtype(int q, int l) { return q == 0 ? 0 : q + gt(l); }
  static constexpr int DP = Plan<L, M, false, 4, 1>::DP;
  static constexpr int mrow(int q, int l) { return Plan<L, M, false, 4, 1>::mrow(q, l); }
  static constexpr int doff(int l) { return Plan<L, M, false, 4, 1>::doff(l); }
  static constexpr int DS = Plan<L, M, false, 4, 1>::DS;
  // B fragments of one K step (kernel-input degree li), grouped by output degree lo:
  // g0, [gate], then (Wr, Wi) for m = 1 .. min(M, li, lo).
  static constexpr int nbl(int li, int lo) { return 1 + gt(lo) + 2 * cmin(cmin(M, li), lo); }
  static constexpr int bbase(int li, int lo) {
    int s = 0;
    for (int k = 0; k < lo; ++k) s += nbl(li, k);
    return s;
  }
  static constexpr int nbfrag(int li) { return bbase(li, L + 1); }
  // MFMAs per row tile and K step summed over li: the schedule's weight of degree lo
  static constexpr int work(int lo) {
    int s = 0;
    for (int li = 0; li <= L; ++li) s += 1 + gt(lo) + 4 * cmin(cmin(M, li), lo);
    return s;
  }
  struct Tab {
    int owner[L + 1];
    int base[L + 1];   // first accumulator slot of degree l in its wave
    int nslots[NW];
  };
  static constexpr Tab make() {
    Tab t{};
    int load[NW] = {};
    bool done[L + 1] = {};
    for (int it = 0; it <= L; ++it) {
      int best = -1;
      for (int l = L; l >= 0; --l)
        if (!done[l] && (best < 0 || work(l) > work(best))) best = l;
      int w = 0;
      for (int k = 1; k < NW; ++k)
        if (load[k] < load[w]) w = k;
      t.owner[best] = w;
      load[w] += work(best);
      done[best] = true;
    }
    for (int w = 0; w < NW; ++w) {
      int s = 0;
      for (int l = 0; l <= L; ++l)
        if (t.owner[l] == w) {
          t.base[l] = s;
          s += RT * ntype(l);
        }
      t.nslots[w] = s;
    }
    return t;
  }
  static constexpr Tab tab = make();
  // B registers of wave w at li: degree lo's fragments start at wboff(w, li, lo)
  static constexpr int wboff(int w, int li, int lo) {
    int s = 0;
    for (int k = 0; k < lo; ++k)
      if (tab.owner[k] == w) s += nbl(li, k);
    return s;
  }
  static constexpr int nbw(int w, int li) { return wboff(w, li, L + 1); }
  static constexpr int NBW = [] {
    int m = 1;
    for (int w = 0; w < NW; ++w) m = nbw(w, L) > m ? nbw(w, L) : m;
    return m;
  }();
  static constexpr int MSLOT = [] {
    int m = 1;
    for (int w = 0; w < NW; ++w) m = tab.nslots[w] > m ? tab.nslots[w] : m;
    return m;
  }();
  // Wigner rows in LDS: the pair-major layout of the dk workspace
  static constexpr int pblk(int l) { return PairLayout<L, M>::pblk(l); }
  static constexpr int woff(int l) { return PairLayout<L, M>::woff(l); }
  static constexpr int WS = PairLayout<L, M>::WS;
  static constexpr int NW4 = (TE * WS / 4 + NT - 1) / NT;  // float4 copies per thread
  // LDS
  static constexpr int A_BYTES = nq(L) * RT * FRAG;      // one A stage
  static constexpr int CH = 16;                           // edges per epilogue chunk
  static constexpr int STG_BYTES = NW * CH * 64 * 4;      // epilogue staging
  static constexpr int U_BYTES = (2 * A_BYTES > STG_BYTES) ? 2 * A_BYTES : STG_BYTES;
  static constexpr int NA = (nq(L) * RT * 64 + NT - 1) / NT;  // A chunks per thread
};

__device__ __forceinline__ uint4 neg_frag(uint4 v, BF16) {
  return make_uint4(v.x ^ 0x80008000u, v.y ^ 0x80008000u, v.z ^ 0x80008000u, v.w ^ 0x80008000u);
}
__device__ __forceinline__ uint4 neg_frag(uint4 v, F32) {
  return make_uint4(v.x ^ 0x80000000u, v.y ^ 0x80000000u, v.z ^ 0x80000000u, v.w ^ 0x80000000u);
}
__device__ __forceinline__ void mfma(f32x16& acc, uint4 a, uint4 b, BF16) {
  bf16x8 av, bv;
  __builtin_memcpy(&av, &a, 16);
  __builtin_memcpy(&bv, &b, 16);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
}
__device__ __forceinline__ void mfma(f32x16& acc, uint4 a, uint4 b, F32) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

template <int L, int M, bool GATE, int NW, int RT, class TM, int MODE>
struct Gemm {
  using P = GPlan<L, M, GATE, NW, RT>;
  static constexpr int TE = P::TE, NT = P::NT, KC = TM::KC, NA = P::NA;
  static constexpr int d = (L + 1) * (L + 1);

  struct Smem {
    alignas(16) float W[TE * P::WS];
    float* optr[TE];  // destination row block of the segment ending at each edge
    int seg[TE];
    int eid[TE];
    alignas(16) char u[P::U_BYTES];
  };

  // ------------------------------------------------------------ A operand
  struct AState {
    int64_t ebase[NA];  // element offset of (edge, row 0, channel half) or -1
    int q[NA];          // row type of the chunk (-1: thread has no chunk)
    int64_t rowoff[NA];
    uint4 reg[NA];
  };

  static __device__ __forceinline__ void a_init(AState& st, const Smem& s, const Args& a, int tid) {
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      const int c = tid + k * NT;
      const int f = c >> 6, ln = c & 63;
      const int q = f / RT, rt = f % RT;
      st.q[k] = (c < P::nq(L) * RT * 64) ? q : -1;
      const int e = rt * 32 + (ln & 31);
      const int ei = (st.q[k] >= 0) ? s.eid[e] : -1;
      st.ebase[k] = ei >= 0 ? static_cast<int64_t>(ei) * P::DP * a.C_k + (ln >> 5) * TM::VEC : -1;
      st.rowoff[k] = 0;
    }
  }
  template <int LI>
  static __device__ __forceinline__ void a_rows(AState& st, const Args& a) {
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      int r = 0;
      static_for<P::nq(LI)>([&](auto Q) {
        if (st.q[k] == decltype(Q)::value) r = P::mrow(decltype(Q)::value, LI);
      });
      st.rowoff[k] = static_cast<int64_t>(r) * a.C_k;
    }
  }
  template <int LI>
  static __device__ __forceinline__ void a_load(AState& st, const Args& a, int ks) {
    const typename TM::raw* y = reinterpret_cast<const typename TM::raw*>(a.a_src);
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      st.reg[k] = make_uint4(0u, 0u, 0u, 0u);
      if (st.q[k] >= 0 && st.q[k] < P::nq(LI) && st.ebase[k] >= 0)
        st.reg[k] = *reinterpret_cast<const uint4*>(y + st.ebase[k] + st.rowoff[k] + ks * KC);
    }
  }
  template <int LI>
  static __device__ __forceinline__ void a_store(const AState& st, Smem& s, int buf, int tid) {
#pragma unroll
    for (int k = 0; k < NA; ++k) {
      const int c = tid + k * NT;
      if (st.q[k] >= 0 && st.q[k] < P::nq(LI))
        *reinterpret_cast<uint4*>(s.u + buf * P::A_BYTES + c * 16) = st.reg[k];
    }
  }

  // ------------------------------------------------------------ B operand
  template <int W, int LI>
  static __device__ __forceinline__ void b_load(uint4 (&b)[P::NBW], const char* wp, int64_t foff,
                                                int ks, int lane) {
    const char* base = wp + (foff + static_cast<int64_t>(ks) * P::nbfrag(LI)) * FRAG + lane * 16;
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::tab.owner[lo] == W) {
        static_for<P::nbl(LI, lo)>([&](auto T) {
          constexpr int t = decltype(T)::value;
          b[P::wboff(W, LI, lo) + t] =
              *reinterpret_cast<const uint4*>(base + (P::bbase(LI, lo) + t) * FRAG);
        });
      }
    });
  }

  // ------------------------------------------------------------ MFMA step
  template <int W, int LI>
  static __device__ __forceinline__ void step(f32x16 (&acc)[P::MSLOT], const char* A,
                                              const uint4 (&b)[P::NBW], int lane) {
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      uint4 af[P::nq(LI)];
      static_for<P::nq(LI)>([&](auto Q) {
        constexpr int q = decltype(Q)::value;
        af[q] = *reinterpret_cast<const uint4*>(A + (q * RT + rt) * FRAG + lane * 16);
      });
      static_for<L + 1>([&](auto LO) {
        constexpr int lo = decltype(LO)::value;
        if constexpr (P::tab.owner[lo] == W) {
          constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
          constexpr int bo = P::wboff(W, LI, lo);
          mfma(acc[sb], af[0], b[bo], TM{});
          if constexpr (P::gt(lo)) mfma(acc[sb + 1], af[0], b[bo + 1], TM{});
          static_for<M>([&](auto MI) {
            constexpr int m = decltype(MI)::value + 1;
            if constexpr (m <= LI && m <= lo) {
              constexpr int bw = bo + 1 + P::gt(lo) + 2 * (m - 1);
              constexpr int sp = sb + P::qtype(2 * m - 1, lo), sm = sb + P::qtype(2 * m, lo);
              const uint4 wr = b[bw], wi = b[bw + 1], nwi = neg_frag(wi, TM{});
              const uint4 ap = af[2 * m - 1], am = af[2 * m];
              if constexpr (MODE == FWD) {
                mfma(acc[sp], ap, wr, TM{});
                mfma(acc[sm], ap, wi, TM{});
                mfma(acc[sp], am, nwi, TM{});
                mfma(acc[sm], am, wr, TM{});
              } else {
                mfma(acc[sp], ap, wr, TM{});
                mfma(acc[sm], ap, nwi, TM{});
                mfma(acc[sp], am, wi, TM{});
                mfma(acc[sm], am, wr, TM{});
              }
            }
          });
        }
      });
    });
  }

  // ------------------------------------------------------------ epilogue
  // Row of register i in row tile rt for lane half h (32x32 accumulator layout).
  static __device__ __forceinline__ int row_of(int rt, int i, int h) {
    return rt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
  }

  template <int lo>
  static __device__ __forceinline__ void bias_gate(f32x16 (&acc)[P::MSLOT], const Args& a,
                                                   int col) {
    static_for<RT>([&](auto RTI) {
      constexpr int sb = P::tab.base[lo] + decltype(RTI)::value * P::ntype(lo);
      if (a.bias != nullptr) {
        const float b0 = a.bias[a.extra + lo * a.C_n + col];
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[sb][i] += b0;
        if constexpr (P::gt(lo)) {
          const float bg = a.bias[(lo - 1) * a.C_n + col];
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[sb + 1][i] += bg;
        }
      }
      if constexpr (GATE) {
        if constexpr (lo == 0) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float z = acc[sb][i];
            acc[sb][i] = z / (1.0f + __expf(-z));
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float g = tanhf(acc[sb + 1][i]);
            static_for<P::nq(lo)>([&](auto Q) {
              constexpr int q = decltype(Q)::value;
              acc[sb + P::qtype(q, lo)][i] *= g;
            });
          }
        }
      }
    });
  }

  // Input gradient: the accumulators hold dY (forward-input side) of degree lo.
  // grad_rad = sum_(+-) dY * R (R: unscaled forward rows); dY *= rad.
  template <int lo>
  static __device__ __forceinline__ void radial(f32x16 (&acc)[P::MSLOT], const Smem& s,
                                                const Args& a, int col, int lane) {
    if (a.rad == nullptr) return;
    const int64_t rw = rad_width<L, M>(a.C_n);
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
      static_for<16>([&](auto II) {
        constexpr int i = decltype(II)::value;
        const int ei = s.eid[row_of(rt, i, lane >> 5)];
        if (ei >= 0) {
          const int64_t eo = static_cast<int64_t>(ei) * rw;
          const typename TM::raw* rp = reinterpret_cast<const typename TM::raw*>(a.rad) + eo;
          const typename TM::raw* rs = reinterpret_cast<const typename TM::raw*>(a.rsave) +
                                       static_cast<int64_t>(ei) * P::DP * a.C_n + col;
          typename TM::raw* dr = reinterpret_cast<typename TM::raw*>(a.drad);
          {
            const int slot = rad_slot<L, M>(0, lo, col, a.C_n);
            const float dy = acc[sb][i];
            if (dr) dr[eo + slot] = TM::cvt(dy * TM::load(rs + P::mrow(0, lo) * a.C_n));
            acc[sb][i] = dy * TM::load(rp + slot);
          }
          static_for<M>([&](auto MI) {
            constexpr int m = decltype(MI)::value + 1;
            if constexpr (m <= lo) {
              constexpr int sp = sb + P::qtype(2 * m - 1, lo), sm = sb + P::qtype(2 * m, lo);
              const int slot = rad_slot<L, M>(2 * m - 1, lo, col, a.C_n);
              const float r = TM::load(rp + slot);
              const float dyp = acc[sp][i], dym = acc[sm][i];
              if (dr)
                dr[eo + slot] = TM::cvt(dyp * TM::load(rs + P::mrow(2 * m - 1, lo) * a.C_n) +
                                        dym * TM::load(rs + P::mrow(2 * m, lo) * a.C_n));
              acc[sp][i] = dyp * r;
              acc[sm][i] = dym * r;
            }
          });
        }
      });
    });
  }

  // Inverse rotation of degree lo and segment sum into out / partials.
  // Per output-column pair p (j = 2p + h for lane half h) and 16-edge chunk:
  // rotate the rows a lane holds (rows of its half), swap halves with
  // v_permlane32_swap so that each lane holds its column j for all 16 rows,
  // run a segmented sum in edge order (uniform selects at segment starts),
  // then store the sums of the segments that end in the chunk.
  template <int W, int lo>
  static __device__ __forceinline__ void rotate_sum(f32x16 (&acc)[P::MSLOT], Smem& s,
                                                    const Args& a, int cb, int wave, int lane,
                                                    uint64_t endmask) {
    constexpr int n = 2 * lo + 1;
    constexpr int nq = P::nq(lo);
    constexpr int PB = P::pblk(lo);
    const int co = lane & 31, h = lane >> 5;
    float* buf = reinterpret_cast<float*>(s.u) + wave * (P::CH * 64);
    const float* Wl = s.W + P::woff(lo);
    const uint64_t startmask = (endmask << 1) | 1ull;
    for (int p = 0; p <= lo; ++p) {
      const bool has_col = 2 * p + h < n;
      const int64_t colo = static_cast<int64_t>(lo * lo + 2 * p + h) * a.C_n + cb * CB + co;
      float run = 0.f;
      static_for<2 * RT>([&](auto CI) {
        constexpr int c = decltype(CI)::value;
        constexpr int rt = c / 2, ib = 8 * (c % 2);
        constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
        float X[8], Y[8];
#pragma unroll
        for (int ii = 0; ii < 8; ++ii) {
          const int i = ib + ii;
          const int e = row_of(rt, i, h);
          const float4* Dp = reinterpret_cast<const float4*>(Wl + e * P::WS + p * PB);
          float dv[PB];
#pragma unroll
          for (int v = 0; v < PB / 4; ++v) {
            const float4 t4 = Dp[v];
            dv[4 * v] = t4.x; dv[4 * v + 1] = t4.y; dv[4 * v + 2] = t4.z; dv[4 * v + 3] = t4.w;
          }
          float v0 = 0.f, v1 = 0.f;
          static_for<nq>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            const float z = acc[sb + P::qtype(q, lo)][i];
            v0 = fmaf(dv[2 * q], z, v0);
            v1 = fmaf(dv[2 * q + 1], z, v1);
          });
          // lanes 32-63 of v0 <-> lanes 0-31 of v1: afterwards lane (co, h) holds
          // column 2p + h, rows of half 0 in v0 and rows of half 1 in v1
          const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(v0), __float_as_uint(v1),
                                                           false, false);
          X[ii] = __uint_as_float(sw[0]);
          Y[ii] = __uint_as_float(sw[1]);
        }
        // chunk rows in edge order: X[0..3], Y[0..3], X[4..7], Y[4..7]
        static_for<P::CH>([&](auto UI) {
          constexpr int u = decltype(UI)::value;
          constexpr int e = c * P::CH + u;
          constexpr int k = 4 * (u >> 3) + (u & 3);
          const float val = ((u >> 2) & 1) ? Y[k] : X[k];
          run = ((startmask >> e) & 1ull) ? val : run + val;
          buf[u * 64 + lane] = run;
        });
        wave_sync();
        uint32_t m = static_cast<uint32_t>(endmask >> (c * P::CH)) & 0xffffu;
        while (m) {
          const int u = __builtin_ctz(m);
          m &= m - 1u;
          const float v = buf[u * 64 + lane];
          float* dst = s.optr[c * P::CH + u];
          if (has_col) dst[colo] = v;
        }
        wave_sync();
      });
    }
  }

  template <int W>
  static __device__ __forceinline__ void body(Smem& s, const Args& a, int cb, int tid, int nvalid) {
    const int wave = tid >> 6, lane = tid & 63;
    f32x16 acc[P::MSLOT];
#pragma unroll
    for (int k = 0; k < P::MSLOT; ++k)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[k][i] = 0.f;

    const int nks = a.C_k / KC;
    const char* wp = a.wpack + static_cast<int64_t>(cb) * a.frags_per_cb * FRAG;
    AState st;
    a_init(st, s, a, tid);
    uint4 bc[P::NBW], bn[P::NBW];
    a_rows<0>(st, a);
    a_load<0>(st, a, 0);
    b_load<W, 0>(bc, wp, 0, 0, lane);
    a_store<0>(st, s, 0, tid);
    __syncthreads();
    int buf = 0;
    int64_t foff = 0;
    static_for<L + 1>([&](auto LIc) {
      constexpr int LI = decltype(LIc)::value;
      for (int ks = 0; ks < nks; ++ks) {
        const bool more = ks + 1 < nks;
        if (more) {
          a_load<LI>(st, a, ks + 1);
          b_load<W, LI>(bn, wp, foff, ks + 1, lane);
        } else if constexpr (LI < L) {
          a_rows<LI + 1>(st, a);
          a_load<LI + 1>(st, a, 0);
          b_load<W, LI + 1>(bn, wp, foff + static_cast<int64_t>(nks) * P::nbfrag(LI), 0, lane);
        }
        step<W, LI>(acc, s.u + buf * P::A_BYTES, bc, lane);
        if (more) {
          a_store<LI>(st, s, buf ^ 1, tid);
        } else if constexpr (LI < L) {
          a_store<LI + 1>(st, s, buf ^ 1, tid);
        }
        __syncthreads();
        buf ^= 1;
#pragma unroll
        for (int k = 0; k < P::NBW; ++k) bc[k] = bn[k];
      }
      foff += static_cast<int64_t>(nks) * P::nbfrag(LI);
    });

    // segment ends of the tile: bit e set if edge e closes its segment
    const int le = lane < TE ? lane : TE - 1, ln = le + 1 < TE ? le + 1 : le;
    const uint64_t endmask = __ballot(lane < nvalid && (lane == nvalid - 1 || s.seg[ln] != s.seg[le]));
    const int col = cb * CB + (lane & 31);
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::tab.owner[lo] == W) {
        if constexpr (MODE == FWD)
          bias_gate<lo>(acc, a, col);
        else
          radial<lo>(acc, s, a, col, lane);
        rotate_sum<W, lo>(acc, s, a, cb, wave, lane, endmask);
      }
    });
  }

  static __device__ __forceinline__ void run(const Args& a) {
    __shared__ Smem s;
    const int tid = threadIdx.x, wave = tid >> 6;
    // XCD-aware mapping: consecutive workgroup ids go round-robin over the 8
    // XCDs.  The n_cb channel-block workgroups of one edge tile are the
    // consecutive workgroups of one XCD, so they run together and read the
    // tile's rows from that XCD's L2 (each XCD holds the weights of all blocks).
    const int64_t bid = blockIdx.x;
    const int64_t slot = bid >> 3;
    const int cb = static_cast<int>(slot % a.n_cb);
    const int64_t tile = (slot / a.n_cb) * 8 + (bid & 7);
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
    // Wigner rows of the tile's edges (pair layout), all loads in flight at once
    {
      constexpr int R4 = P::WS / 4;
      const float4* dk4 = reinterpret_cast<const float4*>(a.dk);
      float4 wv[P::NW4];
#pragma unroll
      for (int k = 0; k < P::NW4; ++k) {
        const int i = tid + k * NT;
        const int e = i / R4, r = i - (i / R4) * R4;
        wv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (i < TE * R4 && s.eid[e] >= 0) wv[k] = dk4[static_cast<int64_t>(s.eid[e]) * R4 + r];
      }
#pragma unroll
      for (int k = 0; k < P::NW4; ++k) {
        const int i = tid + k * NT;
        if (i < TE * R4) reinterpret_cast<float4*>(s.W)[i] = wv[k];
      }
    }
    // Segments cut by the tile boundary go to the partials buffer: the tile's
    // first segment (slot 0) if it began in an earlier tile, its last one
    // (slot 1) if it continues into the next tile.
    const bool fp = (e0 > 0) && (a.seg[e0 - 1] == a.seg[e0]);
    const bool lp = (e0 + nvalid < a.E) && (a.seg[e0 + nvalid] == a.seg[e0 + nvalid - 1]);
    if (tid < TE) {
      float* dst = nullptr;
      if (tid < nvalid) {
        const int sg = s.seg[tid];
        const bool first = sg == s.seg[0], last = sg == s.seg[nvalid - 1];
        if ((first && fp) || (last && lp))
          dst = a.part + (tile * 2 + (first ? 0 : 1)) * d * a.C_n;
        else
          dst = a.out + static_cast<int64_t>(sg) * d * a.C_n;
      }
      s.optr[tid] = dst;
    }
    static_for<NW>([&](auto WI) {
      constexpr int w = decltype(WI)::value;
      if (wave == w) body<w>(s, a, cb, tid, nvalid);
    });
  }
};

template <int L, int M, bool GATE, int NW, int RT, class TM, int MODE>
__global__ __launch_bounds__(NW * 64, 2) void gemm_kernel(Args a) {
  Gemm<L, M, GATE, NW, RT, TM, MODE>::run(a);
}

}  // namespace msg
}  // namespace maloq
