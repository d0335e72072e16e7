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
//     in the exact lane order of the MFMA A operand, copied global -> LDS by
//     DMA (global_load_lds) into a ring of three stages, two steps ahead; one
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

// MODE FWD: a gated block has one more output row type per degree l >= 1 (the
// gate pre-activations); MODE BWD_DX: one more input row type per degree
// l >= 1 (dL/dgate), whose products with the transposed gate weights add to
// the m = 0 outputs.
template <int L, int M, bool GATE, int NW, int RT, int MODE = 0>
struct GPlan {
  static constexpr int TE = 32 * RT;
  static constexpr int NT = NW * 64;
  static_assert(TE <= 64, "segment masks are 64-bit");
  static constexpr bool BWD = MODE == 1 || MODE == 3;  // BWD_DX, BWD_EDGE
  static constexpr int gt(int l) { return (GATE && !BWD && l >= 1) ? 1 : 0; }   // output gate row
  static constexpr int gin(int l) { return (GATE && BWD && l >= 1) ? 1 : 0; }   // input gate row
  static constexpr int nq(int l) { return 1 + 2 * cmin(M, l); }
  static constexpr int nqa(int l) { return nq(l) + gin(l); }  // A row types of input degree l
  // Gate rows apart (GW): a gated forward on 8 waves (lmax 6) puts the gate
  // row of each degree l >= 1 in the wave with the fewest accumulators at that
  // point (the wave left without a degree, then those of the light degrees),
  // so the waves of the heavy degrees hold only their kept rows; the gate
  // values reach a degree's wave through LDS after the K loop.
  static constexpr bool GW = GATE && !BWD && NW == 8;
  static constexpr int gacc(int l) { return GW ? 0 : gt(l); }  // gate row among degree l's accumulators
  static constexpr int ntype(int l) { return nq(l) + gacc(l); }
  // accumulator type of row type q of degree l (0: m=0, [1: gate], then +1, -1, +2, ...)
  static constexpr int qtype(int q, int l) { return q == 0 ? 0 : q + gacc(l); }
  static constexpr int DP = Plan<L, M, false, 4, 1>::DP;
  static constexpr int DPA = DP + ((GATE && BWD) ? L : 0);  // A rows per edge
  // A-source row of input row type q of degree l (gate rows follow the kept rows)
  static constexpr int arow(int q, int l) { return q < nq(l) ? Plan<L, M, false, 4, 1>::mrow(q, l) : DP + l - 1; }
  static constexpr int mrow(int q, int l) { return Plan<L, M, false, 4, 1>::mrow(q, l); }
  static constexpr int doff(int l) { return Plan<L, M, false, 4, 1>::doff(l); }
  static constexpr int DS = Plan<L, M, false, 4, 1>::DS;
  // B fragments of one K step (kernel-input degree li), grouped by output degree lo:
  // g0, [gate], then (Wr, Wi) for m = 1 .. min(M, li, lo).
  static constexpr int nbl(int li, int lo) { return 1 + gt(lo) + gin(li) + 2 * cmin(cmin(M, li), lo); }
  static constexpr int bbase(int li, int lo) {
    int s = 0;
    for (int k = 0; k < lo; ++k) s += nbl(li, k);
    return s;
  }
  static constexpr int nbfrag(int li) { return bbase(li, L + 1); }
  // B registers of degree lo at li in its own wave (with GW the gate fragment
  // is the gate wave's), and the packed position of that wave's fragment t
  static constexpr int nblr(int li, int lo) { return nbl(li, lo) - gt(lo) + gacc(lo); }
  static constexpr int bpos(int lo, int t) { return t == 0 ? 0 : t + gt(lo) - gacc(lo); }
  // MFMAs per row tile and K step summed over li: the schedule's weight of degree lo
  static constexpr int work(int lo) {
    int s = 0;
    for (int li = 0; li <= L; ++li) s += 1 + gacc(lo) + gin(li) + 4 * cmin(cmin(M, li), lo);
    return s;
  }
  struct Tab {
    int owner[L + 1];
    int base[L + 1];   // first accumulator slot of degree l in its wave
    int nslots[NW];
    int gowner[L + 1];  // GW: wave holding the gate row of degree l >= 1
    int gbase[L + 1];   // GW: its accumulator slots gbase .. gbase + RT - 1 (one per row tile)
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
    if (GW)
      for (int l = 1; l <= L; ++l) {
        int w = 0;
        for (int k = 1; k < NW; ++k)
          if (t.nslots[k] < t.nslots[w]) w = k;
        t.gowner[l] = w;
        t.gbase[l] = t.nslots[w];
        t.nslots[w] += RT;
      }
    return t;
  }
  static constexpr Tab tab = make();
  static constexpr bool gown(int w, int l) { return GW && l >= 1 && tab.gowner[l] == w; }
  static constexpr bool has_deg(int w) {
    for (int l = 0; l <= L; ++l)
      if (tab.owner[l] == w) return true;
    return false;
  }
  // B registers of wave w at li: degree lo's fragments start at wboff(w, li, lo),
  // then (GW) the gate fragment of each gate row it holds, at gboff(w, li, lo)
  static constexpr int wboff(int w, int li, int lo) {
    int s = 0;
    for (int k = 0; k < lo; ++k)
      if (tab.owner[k] == w) s += nblr(li, k);
    return s;
  }
  static constexpr int gboff(int w, int li, int lo) {
    int s = wboff(w, li, L + 1);
    for (int k = 1; k < lo; ++k)
      if (gown(w, k)) ++s;
    return s;
  }
  static constexpr int nbw(int w, int li) { return gboff(w, li, L + 1); }
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
  // Wigner rows in LDS: TE WS / 4 16-byte chunks, copied by DMA in whole
  // 64-lane instructions (the array is padded to a multiple of 64 chunks)
  static constexpr int W16 = TE * WS / 4;
  static constexpr int W16P = (W16 + 63) / 64 * 64;
  // LDS
  static constexpr int A_BYTES = nqa(L) * RT * FRAG;     // one A stage
  static constexpr int CH = 16;                           // edges per epilogue chunk
  static constexpr int NA = (nqa(L) * RT * 64 + NT - 1) / NT;  // A chunks per thread
};

// One lane's 16 bytes of an MFMA operand fragment (a native vector, so that
// arrays of fragments are promoted to registers).
typedef unsigned int frag_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ frag_t neg_frag(frag_t v, BF16) { return v ^ 0x80008000u; }
__device__ __forceinline__ frag_t neg_frag(frag_t v, F32) { return v ^ 0x80000000u; }
__device__ __forceinline__ void mfma(f32x16& acc, frag_t a, frag_t b, BF16) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16((bf16x8)a, (bf16x8)b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mfma(f32x16& acc, frag_t a, frag_t b, F32) {
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.x), __uint_as_float(b.x), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.y), __uint_as_float(b.y), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.z), __uint_as_float(b.z), acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(__uint_as_float(a.w), __uint_as_float(b.w), acc, 0, 0, 0);
}

template <int L, int M, bool GATE, int NW, int RT, class TM, int MODE>
struct Gemm {
  using P = GPlan<L, M, GATE, NW, RT, MODE>;
  static constexpr int TE = P::TE, NT = P::NT, KC = TM::KC;
  static constexpr int d = (L + 1) * (L + 1);

  struct Smem {
    float* optr[TE];  // destination row block of the segment ending at each edge
    int seg[TE];
    int eid[TE];
  };
  // A stages (three distinct LDS objects, so the compiler can tell a stage
  // being filled by DMA from the one being read); after the K loop they hold
  // the epilogue's per-wave staging, WPS waves per stage (2 of 4 waves: st0
  // and st1; 3 of 8 waves: all three).
  // per-wave epilogue staging: the 16-edge scan chunk or the 32 x 36 transpose tile
  static constexpr int PW = (P::CH * 64 > 32 * 36 ? P::CH * 64 : 32 * 36) * 4;
  static constexpr int WPS = (NW + 2) / 3;
  // Gate wave (P::GW): after the K loop the stages also carry tanh of the gate
  // rows to the degree waves, degree l's RT x 16 x 64 floats in stage (l - 1) / GPS.
  static constexpr int GPS = (L + 2) / 3;
  static constexpr int GXB = P::GW ? GPS * RT * 16 * 64 * 4 : 0;
  static constexpr int SB0 = (P::A_BYTES > WPS * PW) ? P::A_BYTES : WPS * PW;
  static constexpr int SB = SB0 > GXB ? SB0 : GXB;
  static __device__ __forceinline__ float* wave_staging(int wave, char* st0, char* st1, char* st2) {
    const int k = wave / WPS;
    return reinterpret_cast<float*>((k == 0 ? st0 : (k == 1 ? st1 : st2)) + (wave - k * WPS) * PW);
  }
  typedef __attribute__((address_space(3))) void lds_void;

  // ------------------------------------------------------------ A operand
  // A staging: the nq(L) RT fragments of a K step are split over the waves,
  // waves with the least MFMA work taking the most (their registers are free);
  // wave W stages the fragments f with stager(f) == W, k-th of them in slot k.
  // Row type q = f / RT, row tile f % RT; lane (row, half) copies 16 bytes of
  // its edge's row.  Which fragments exist is a compile-time property of
  // (W, k, LI), so every load is unconditional (which keeps the compiler's
  // vmcnt accounting exact); lanes of edges beyond the tile read the tile's
  // first edge, whose rows in those accumulator lanes are never stored.
  struct ATab {
    int frag[NW][P::nqa(L) * RT];
    int count[NW];
  };
  static constexpr ATab make_atab() {
    ATab t{};
    int order[NW] = {};
    for (int w = 0; w < NW; ++w) order[w] = w;
    for (int i = 0; i < NW; ++i)  // waves by ascending MFMA slots
      for (int j = i + 1; j < NW; ++j)
        if (P::tab.nslots[order[j]] < P::tab.nslots[order[i]]) {
          const int x = order[i];
          order[i] = order[j];
          order[j] = x;
        }
    constexpr int F = P::nqa(L) * RT;
    for (int f = 0; f < F; ++f) {
      int best = order[0];  // fewest staged so far, ties to the lighter wave
      for (int i = 1; i < NW; ++i) {
        const int w = order[i];
        const int cb = t.count[best] - (best == order[0] ? (F + NW - 1) / NW - F / NW : 0);
        const int cw = t.count[w] - (w == order[0] ? (F + NW - 1) / NW - F / NW : 0);
        if (cw < cb) best = w;
      }
      t.frag[best][t.count[best]++] = f;
    }
    return t;
  }
  static constexpr ATab atab = make_atab();
  static constexpr int NAW = [] {
    int m = 1;
    for (int w = 0; w < NW; ++w) m = atab.count[w] > m ? atab.count[w] : m;
    return m;
  }();
  template <int W, int k>
  static constexpr int afrag() { return atab.frag[W][k]; }
  template <int W, int k, int LI>
  static constexpr bool avalid() { return k < atab.count[W] && afrag<W, k>() < P::nqa(LI) * RT; }

  struct AState {
    int64_t ebase[NAW];  // element offset of (edge, row 0, channel half)
  };

  template <int W>
  static __device__ __forceinline__ void a_init(AState& st, const Smem& s, const Args& a, int lane) {
    static_for<NAW>([&](auto K) {
      constexpr int k = decltype(K)::value;
      if constexpr (k >= atab.count[W]) return;
      constexpr int rt = afrag<W, k>() % RT;
      const int e = rt * 32 + (lane & 31);
      const int ei = s.eid[e] >= 0 ? s.eid[e] : s.eid[0];
      st.ebase[k] = static_cast<int64_t>(ei) * P::DPA * a.C_k + (lane >> 5) * TM::VEC;
    });
  }
  // Direct global -> LDS copies of this wave's fragments of step (LI, ks):
  // lane i's 16 bytes land at stage + f*FRAG + 16 i, the MFMA lane order.
  template <int W, int LI>
  static __device__ __forceinline__ void a_dma(const AState& st, char* stage, const Args& a, int ks) {
    const typename TM::raw* y = reinterpret_cast<const typename TM::raw*>(a.a_src);
    static_for<NAW>([&](auto K) {
      constexpr int k = decltype(K)::value;
      if constexpr (avalid<W, k, LI>()) {
        constexpr int q = afrag<W, k>() / RT;
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass does not know gfx950's 16-byte form
        __builtin_amdgcn_global_load_lds(
            y + st.ebase[k] + static_cast<int64_t>(P::arow(q, LI)) * a.C_k + ks * KC,
            (lds_void*)(stage + afrag<W, k>() * FRAG), 16, 0, 0);
#endif
      }
    });
  }

  // ------------------------------------------------------------ B operand
  template <int W, int LI>
  static __device__ __forceinline__ void b_load(frag_t (&b)[P::NBW], const char* wp, int64_t foff,
                                                int ks, int lane) {
    const char* base = wp + (foff + static_cast<int64_t>(ks) * P::nbfrag(LI)) * FRAG + lane * 16;
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::tab.owner[lo] == W) {
        static_for<P::nblr(LI, lo)>([&](auto T) {
          constexpr int t = decltype(T)::value;
          b[P::wboff(W, LI, lo) + t] =
              *reinterpret_cast<const frag_t*>(base + (P::bbase(LI, lo) + P::bpos(lo, t)) * FRAG);
        });
      }
    });
    static_for<L + 1>([&](auto LO) {  // a gate fragment follows its degree's m = 0 fragment
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::gown(W, lo))
        b[P::gboff(W, LI, lo)] = *reinterpret_cast<const frag_t*>(base + (P::bbase(LI, lo) + 1) * FRAG);
    });
  }

  // ------------------------------------------------------------ MFMA step
  // Fragment (row type q, all row tiles) of the current stage.
  template <int q>
  static __device__ __forceinline__ void read_q(frag_t (&af)[RT], const char* A, int lane) {
    static_for<RT>([&](auto R) {
      constexpr int rt = decltype(R)::value;
      af[rt] = *reinterpret_cast<const frag_t*>(A + (q * RT + rt) * FRAG + lane * 16);
    });
  }
  // m = 0 (and gate) products of every owned degree: forward, the gate
  // outputs from the m = 0 inputs; input gradient, the m = 0 outputs also
  // from the gate-gradient inputs ag.
  template <int W, int LI>
  static __device__ __forceinline__ void mma_m0(f32x16 (&acc)[P::MSLOT], const frag_t (&a0)[RT],
                                                const frag_t (&ag)[RT], const frag_t (&b)[P::NBW]) {
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::gown(W, lo))
        static_for<RT>([&](auto R) {
          constexpr int rt = decltype(R)::value;
          mfma(acc[P::tab.gbase[lo] + rt], a0[rt], b[P::gboff(W, LI, lo)], TM{});
        });
    });
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::tab.owner[lo] == W) {
        constexpr int bo = P::wboff(W, LI, lo);
        static_for<RT>([&](auto R) {
          constexpr int rt = decltype(R)::value;
          constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
          mfma(acc[sb], a0[rt], b[bo], TM{});
          if constexpr (P::gacc(lo)) mfma(acc[sb + 1], a0[rt], b[bo + 1], TM{});
          if constexpr (P::gin(LI)) mfma(acc[sb], ag[rt], b[bo + 1], TM{});
        });
      }
    });
  }
  // +-m products of every owned degree.  Forward: y+ += Wr x+ - Wi x-,
  // y- += Wi x+ + Wr x-; input gradient: dx+ += Wr dy+ + Wi dy-,
  // dx- += -Wi dy+ + Wr dy-.  The negated Wi is formed after the last use of Wi.
  template <int W, int LI, int m>
  static __device__ __forceinline__ void mma_m(f32x16 (&acc)[P::MSLOT], const frag_t (&ap)[RT],
                                               const frag_t (&am)[RT], const frag_t (&b)[P::NBW]) {
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::tab.owner[lo] == W && m <= lo) {
        constexpr int bw = P::wboff(W, LI, lo) + 1 + P::gacc(lo) + P::gin(LI) + 2 * (m - 1);
        const frag_t wr = b[bw], wi = b[bw + 1];
        static_for<RT>([&](auto R) {
          constexpr int rt = decltype(R)::value;
          constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
          constexpr int sp = sb + P::qtype(2 * m - 1, lo), sm = sb + P::qtype(2 * m, lo);
          if constexpr (!P::BWD) {
            mfma(acc[sm], ap[rt], wi, TM{});
            mfma(acc[sm], am[rt], wr, TM{});
            mfma(acc[sp], ap[rt], wr, TM{});
          } else {
            mfma(acc[sp], ap[rt], wr, TM{});
            mfma(acc[sp], am[rt], wi, TM{});
            mfma(acc[sm], am[rt], wr, TM{});
          }
        });
        const frag_t nwi = neg_frag(wi, TM{});
        static_for<RT>([&](auto R) {
          constexpr int rt = decltype(R)::value;
          constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
          if constexpr (!P::BWD)
            mfma(acc[sb + P::qtype(2 * m - 1, lo)], am[rt], nwi, TM{});
          else
            mfma(acc[sb + P::qtype(2 * m, lo)], ap[rt], nwi, TM{});
        });
      }
    });
  }

  // DMA instructions wave W issues for one K step of input degree LI.
  template <int W, int LI>
  static constexpr int ndma() {
    int n = 0;
    for (int k = 0; k < NAW; ++k)
      if (k < atab.count[W] && atab.frag[W][k] < P::nqa(LI) * RT) ++n;
    return n;
  }
  template <int I>
  static __device__ __forceinline__ char* stage(char* s0, char* s1, char* s2) {
    return I == 0 ? s0 : (I == 1 ? s1 : s2);
  }

  // One K step of wave W on input degree LI: A fragments from stage RD, B
  // fragments in bn (loaded by the previous step).  The A stages form a ring of
  // three, filled by DMA two steps ahead; B is loaded one step ahead.  At entry
  // the wave's outstanding vector-memory operations are, in issue order, the B
  // loads of this step and the DMA of the next step (PEND instructions), so
  // vmcnt(PEND) leaves only the latter in flight, and after the barrier every
  // wave's DMA of this step has landed.  lgkmcnt(0): the previous step's LDS
  // reads are complete before any wave refills that stage.  Then: B of the
  // next step (degree NB, K step ksb, fragment base fb; none if NB < 0) into
  // bn, DMA of the step after it (degree NA, K step ksa; none if NA < 0) into
  // stage (RD + 2) % 3, and the MFMAs of this step.
  template <int W, int LI, int RD, int NB, int NA, int PEND>
  static __device__ __forceinline__ void kstep(f32x16 (&acc)[P::MSLOT], frag_t (&bn)[P::NBW],
                                               const AState& st, char* s0, char* s1, char* s2,
                                               const Args& a, const char* wp, int64_t fb, int ksb,
                                               int ksa, int lane) {
    // s_waitcnt as a builtin, so that the compiler's own wait insertion counts it
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((PEND & 15) | (7 << 4) | ((PEND >> 4) << 14));  // vmcnt(PEND) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    frag_t bc[P::NBW];
#pragma unroll
    for (int i = 0; i < P::NBW; ++i) bc[i] = bn[i];
    if constexpr (NB >= 0) b_load<W, NB>(bn, wp, fb, ksb, lane);
    if constexpr (NA >= 0) a_dma<W, NA>(st, stage<(RD + 2) % 3>(s0, s1, s2), a, ksa);
    // keep the next steps' loads ahead of this step's MFMAs
    __builtin_amdgcn_sched_barrier(0);
    const char* rd = stage<RD>(s0, s1, s2);
    frag_t a0[RT], ag[RT];
    read_q<0>(a0, rd, lane);
    if constexpr (P::gin(LI)) read_q<P::nq(LI)>(ag, rd, lane);
    mma_m0<W, LI>(acc, a0, ag, bc);
    static_for<M>([&](auto MI) {
      constexpr int m = decltype(MI)::value + 1;
      if constexpr (m <= LI && P::has_deg(W)) {
        frag_t ap[RT], am[RT];
        read_q<2 * m - 1>(ap, rd, lane);
        read_q<2 * m>(am, rd, lane);
        mma_m<W, LI, m>(acc, ap, am, bc);
      }
    });
  }

  // The nks K steps of input degree LI.  KR = nks % 3 for nks >= 2 (then the
  // stage of the degree's first step is (LI nks) % 3 = (LI KR) % 3), KR = 3 for
  // nks == 1.  Step ks loads B of ks + 1 and DMAs ks + 2, crossing into degree
  // LI + 1 for the last two steps; the ring position of every step is static.
  template <int W, int LI, int KR>
  static __device__ __forceinline__ void kdegree(f32x16 (&acc)[P::MSLOT], frag_t (&bn)[P::NBW],
                                                 const AState& st, char* s0, char* s1, char* s2,
                                                 const Args& a, const char* wp, int64_t foff, int nks,
                                                 int lane) {
    constexpr int NXT = LI < L ? LI + 1 : -1;
    constexpr int ND = ndma<W, LI>();
    if constexpr (KR == 3) {  // one step per degree: B of degree LI + 1, DMA of LI + 2
      constexpr int NA = LI + 2 <= L ? LI + 2 : -1;
      constexpr int PEND = NXT >= 0 ? ndma<W, (NXT >= 0 ? NXT : 0)>() : 0;
      kstep<W, LI, LI % 3, NXT, NA, PEND>(acc, bn, st, s0, s1, s2, a, wp, foff + P::nbfrag(LI), 0, 0, lane);
    } else {
      constexpr int PH = (LI * KR) % 3;
      constexpr int REM = (KR + 1) % 3;  // (nks - 2) % 3
      int ks = 0;
      for (; ks + 3 <= nks - 2; ks += 3) {
        kstep<W, LI, PH, LI, LI, ND>(acc, bn, st, s0, s1, s2, a, wp, foff, ks + 1, ks + 2, lane);
        kstep<W, LI, (PH + 1) % 3, LI, LI, ND>(acc, bn, st, s0, s1, s2, a, wp, foff, ks + 2, ks + 3, lane);
        kstep<W, LI, (PH + 2) % 3, LI, LI, ND>(acc, bn, st, s0, s1, s2, a, wp, foff, ks + 3, ks + 4, lane);
      }
      if constexpr (REM >= 1)
        kstep<W, LI, PH, LI, LI, ND>(acc, bn, st, s0, s1, s2, a, wp, foff, ks + 1, ks + 2, lane);
      if constexpr (REM >= 2)
        kstep<W, LI, (PH + 1) % 3, LI, LI, ND>(acc, bn, st, s0, s1, s2, a, wp, foff, ks + 2, ks + 3, lane);
      constexpr int PEND_NXT = NXT >= 0 ? ndma<W, (NXT >= 0 ? NXT : 0)>() : 0;
      const int64_t fnext = foff + static_cast<int64_t>(nks) * P::nbfrag(LI);
      // ks = nks - 2: B of (LI, nks - 1), DMA of (LI + 1, 0)
      kstep<W, LI, (PH + REM) % 3, LI, NXT, ND>(acc, bn, st, s0, s1, s2, a, wp, foff, nks - 1, 0, lane);
      // ks = nks - 1: B of (LI + 1, 0), DMA of (LI + 1, 1)
      kstep<W, LI, (PH + REM + 1) % 3, NXT, NXT, PEND_NXT>(acc, bn, st, s0, s1, s2, a, wp, fnext, 0, 1,
                                                            lane);
    }
  }

  // ------------------------------------------------------------ epilogue
  // Row of register i in row tile rt for lane half h (32x32 accumulator layout).
  static __device__ __forceinline__ int row_of(int rt, int i, int h) {
    return rt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
  }

  template <int lo>
  static __device__ __forceinline__ void add_bias(f32x16 (&acc)[P::MSLOT], const Args& a, int col) {
    static_for<RT>([&](auto RTI) {
      constexpr int sb = P::tab.base[lo] + decltype(RTI)::value * P::ntype(lo);
      // branch-free: a runtime branch around accumulator updates costs spills
      const float b0 = a.bias != nullptr ? a.bias[a.extra + lo * a.C_n + col] : 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[sb][i] += b0;
      if constexpr (P::gacc(lo)) {
        const float bg = a.bias != nullptr ? a.bias[(lo - 1) * a.C_n + col] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[sb + 1][i] += bg;
      }
    });
  }

  // Gated forward: the pre-activation rows of degree lo (kept rows and the gate
  // row) to a.gsave [edge id][d' + L][C_n], each 32 x 32 block transposed
  // through the wave's LDS tile so that a lane stores 16 channels of one edge.
  // ZOUT: the activated kept rows (no gate rows) to a.zout [edge id][d'][C_n]
  // instead (the edge-frame output of FWD_EDGE).
  template <int lo, bool ZOUT = false>
  static __device__ __forceinline__ void save_pre(const f32x16 (&acc)[P::MSLOT], const Smem& s,
                                                  const Args& a, int cb, float* tb, int lane) {
    const int co = lane & 31, h = lane >> 5;
    constexpr int RPE = ZOUT ? P::DP : P::DP + L;  // rows per edge of the destination
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
      const int ei = s.eid[rt * 32 + co];
      typename TM::raw* g = reinterpret_cast<typename TM::raw*>(ZOUT ? a.zout : a.gsave) +
                            static_cast<int64_t>(ei >= 0 ? ei : 0) * RPE * a.C_n + cb * CB + 16 * h;
      static_for<P::ntype(lo)>([&](auto TI) {
        constexpr int t = decltype(TI)::value;  // accumulator type: 0, [gate], +1, -1, ...
        if constexpr (ZOUT && P::gacc(lo) && t == 1) return;
        constexpr int row = (P::gacc(lo) && t == 1) ? P::DP + lo - 1
                                                    : P::mrow(t == 0 ? 0 : t - P::gacc(lo), lo);
        store_block(acc[sb + t], g, ei, row, a.C_n, tb, co, h);
      });
    });
  }

  // One 32-edge x 32-channel accumulator block v to row `row` of each edge's
  // destination rows g (lane (co, h): edge co, channels 16h..16h+15; nothing
  // for ei < 0), transposed through the wave's LDS tile tb.
  static __device__ __forceinline__ void store_block(const f32x16& v, typename TM::raw* g, int ei, int row,
                                                     int64_t C_n, float* tb, int co, int h) {
#pragma unroll
    for (int i = 0; i < 16; ++i) tb[tsw(8 * (i >> 2) + 4 * h + (i & 3), co)] = v[i];
    wave_sync();
    if (ei >= 0) {
      float w[16];
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const float4 t4 = *reinterpret_cast<const float4*>(tb + tsw(co, 16 * h + 4 * g4));
        w[4 * g4] = t4.x; w[4 * g4 + 1] = t4.y; w[4 * g4 + 2] = t4.z; w[4 * g4 + 3] = t4.w;
      }
      float w8[8];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int k = 0; k < 8; ++k) w8[k] = w[8 * half + k];
        store_vec<TM, 8>(g + static_cast<int64_t>(row) * C_n + 8 * half, w8);
      }
    }
    wave_sync();
  }

  // ---- gate rows apart (P::GW): wave tab.gowner[l] holds the gate row of
  // degree l, row tile rt, in accumulator tab.gbase[l] + rt.
  // Gate bias, then (with a.gsave) the pre-activation gate rows to a.gsave
  // [edge id][d' + L][C_n], row d' + l - 1.
  template <int W>
  static __device__ __forceinline__ void gate_rows(f32x16 (&acc)[P::MSLOT], const Smem& s, const Args& a,
                                                   int cb, float* tb, int lane) {
    const int co = lane & 31, h = lane >> 5, col = cb * CB + co;
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::gown(W, lo)) {
        const float bg = a.bias != nullptr ? a.bias[(lo - 1) * a.C_n + col] : 0.f;
        static_for<RT>([&](auto R) {
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[P::tab.gbase[lo] + decltype(R)::value][i] += bg;
        });
      }
    });
    if (a.gsave == nullptr) return;
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      const int ei = s.eid[rt * 32 + co];
      typename TM::raw* gp = reinterpret_cast<typename TM::raw*>(a.gsave) +
                             static_cast<int64_t>(ei >= 0 ? ei : 0) * (P::DP + L) * a.C_n + cb * CB + 16 * h;
      static_for<L + 1>([&](auto LO) {
        constexpr int lo = decltype(LO)::value;
        if constexpr (P::gown(W, lo)) store_block(acc[P::tab.gbase[lo] + rt], gp, ei, P::DP + lo - 1, a.C_n, tb, co, h);
      });
    });
  }
  // tanh of the gate row of degree g + 1, row tile rt: register i of lane at
  // gx<g, rt>[i * 64 + lane]
  template <int g, int rt>
  static __device__ __forceinline__ float* gx(char* st0, char* st1, char* st2) {
    constexpr int k = g / GPS;
    return reinterpret_cast<float*>(k == 0 ? st0 : (k == 1 ? st1 : st2)) + ((g % GPS) * RT + rt) * 16 * 64;
  }
  template <int W>
  static __device__ __forceinline__ void gate_out(const f32x16 (&acc)[P::MSLOT], char* st0, char* st1,
                                                  char* st2, int lane) {
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::gown(W, lo))
        static_for<RT>([&](auto R) {
          constexpr int rt = decltype(R)::value;
          float* x = gx<lo - 1, rt>(st0, st1, st2);
#pragma unroll
          for (int i = 0; i < 16; ++i) x[i * 64 + lane] = tanhf(acc[P::tab.gbase[lo] + rt][i]);
        });
    });
  }
  // A degree's GateActivation with the gate values from LDS.
  template <int lo>
  static __device__ __forceinline__ void gate_act_gw(f32x16 (&acc)[P::MSLOT], char* st0, char* st1,
                                                     char* st2, int lane) {
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
      if constexpr (lo == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float z = acc[sb][i];
          acc[sb][i] = z / (1.0f + __expf(-z));
        }
      } else {
        const float* x = gx<lo - 1, rt>(st0, st1, st2);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float g = x[i * 64 + lane];
          static_for<P::nq(lo)>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            acc[sb + P::qtype(q, lo)][i] *= g;
          });
        }
      }
    });
  }

  // BWD_EDGE with a.gsave: the GateActivation backward (activation.py:57-77)
  // fused into the edge-frame store.  acc holds o = dL/d(gate output) of degree
  // lo; after the transpose through LDS a lane holds 16 channels of one edge,
  // reads the saved pre-activations z of the same row (and the gate row) and
  // writes to a.zout [edge id][d' + L][C_n]:
  //   lo = 0:  dpre = o s (1 + z (1 - s)),  s = sigmoid(z);
  //   lo >= 1: t = tanh(z_gate); dpre_q = o_q t;  dgate = (1 - t^2) sum_q o_q z_q.
  template <int lo>
  static __device__ __forceinline__ void store_gate_bwd(const f32x16 (&acc)[P::MSLOT], const Smem& s,
                                                        const Args& a, int cb, float* tb, int lane) {
    constexpr int DG = P::DP + L;
    const int co = lane & 31, h = lane >> 5;
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
      const int ei = s.eid[rt * 32 + co];
      const int64_t base = static_cast<int64_t>(ei >= 0 ? ei : 0) * DG * a.C_n + cb * CB + 16 * h;
      typename TM::raw* g = reinterpret_cast<typename TM::raw*>(a.zout) + base;
      const typename TM::raw* zs = reinterpret_cast<const typename TM::raw*>(a.gsave) + base;
      float tg[16], dg[16];
      if constexpr (lo > 0) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          tg[k] = 0.f;
          dg[k] = 0.f;
        }
        if (ei >= 0) {
          float t8[8];
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            load_vec<TM, 8>(zs + static_cast<int64_t>(P::DP + lo - 1) * a.C_n + 8 * half, t8);
#pragma unroll
            for (int k = 0; k < 8; ++k) tg[8 * half + k] = tanhf(t8[k]);
          }
        }
      }
      static_for<P::ntype(lo)>([&](auto TI) {
        constexpr int t = decltype(TI)::value;
        constexpr int row = P::mrow(t, lo);
#pragma unroll
        for (int i = 0; i < 16; ++i) tb[tsw(8 * (i >> 2) + 4 * h + (i & 3), co)] = acc[sb + t][i];
        wave_sync();
        if (ei >= 0) {
          float v[16];
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const float4 t4 = *reinterpret_cast<const float4*>(tb + tsw(co, 16 * h + 4 * g4));
            v[4 * g4] = t4.x; v[4 * g4 + 1] = t4.y; v[4 * g4 + 2] = t4.z; v[4 * g4 + 3] = t4.w;
          }
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            float z8[8], w8[8];
            load_vec<TM, 8>(zs + static_cast<int64_t>(row) * a.C_n + 8 * half, z8);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float o = v[8 * half + k], z = z8[k];
              if constexpr (lo == 0) {
                const float sg = 1.0f / (1.0f + expf(-z));
                w8[k] = o * (sg * (1.0f + z * (1.0f - sg)));
              } else {
                dg[8 * half + k] = fmaf(o, z, dg[8 * half + k]);
                w8[k] = o * tg[8 * half + k];
              }
            }
            store_vec<TM, 8>(g + static_cast<int64_t>(row) * a.C_n + 8 * half, w8);
          }
        }
        wave_sync();
      });
      if constexpr (lo > 0) {
        if (ei >= 0) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            float w8[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float tv = tg[8 * half + k];
              w8[k] = dg[8 * half + k] * (1.0f - tv * tv);
            }
            store_vec<TM, 8>(g + static_cast<int64_t>(P::DP + lo - 1) * a.C_n + 8 * half, w8);
          }
        }
      }
    });
  }

  template <int lo>
  static __device__ __forceinline__ void gate_act(f32x16 (&acc)[P::MSLOT]) {
    static_for<RT>([&](auto RTI) {
      constexpr int sb = P::tab.base[lo] + decltype(RTI)::value * P::ntype(lo);
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
  // Each 32-edge x 32-channel block of dY is transposed through a per-wave
  // LDS tile (pitch 36 floats: 16-byte rows, at most 2-way bank conflicts) into row layout, where lane (edge r,
  // half h) holds channels 16h..16h+15 of one edge: R, rad and grad_rad then
  // move as 32- or 64-byte vectors per lane; the scaled block is transposed
  // back for the inverse rotation.
  static __device__ __forceinline__ int tsw(int r, int c) { return r * 36 + c; }

  template <int lo>
  static __device__ __forceinline__ void radial(f32x16 (&acc)[P::MSLOT], const Smem& s,
                                                const Args& a, int cb, float* tb, int lane) {
    const int64_t rw = rad_width<L, M>(a.C_n);
    const int co = lane & 31, h = lane >> 5;
    const int c0 = cb * CB + h * 16;  // first channel of this lane in row layout
    constexpr int VEC = TM::VEC;      // channels per 16-byte piece
    constexpr int NU = 16 / VEC;      // 16-byte pieces per 16 channels
    static_for<RT>([&](auto RTI) {
      constexpr int rt = decltype(RTI)::value;
      constexpr int sb = P::tab.base[lo] + rt * P::ntype(lo);
      const int ei = s.eid[rt * 32 + co];
      const int64_t eis = ei >= 0 ? ei : s.eid[0];
      const typename TM::raw* rsave = reinterpret_cast<const typename TM::raw*>(a.rsave) +
                                      eis * P::DP * a.C_n + c0;
      static_for<1 + (lo < M ? lo : M)>([&](auto MI) {
        constexpr int m = decltype(MI)::value;
        constexpr int q0 = m == 0 ? 0 : 2 * m - 1, nqm = m == 0 ? 1 : 2;
        const typename TM::raw* radp = reinterpret_cast<const typename TM::raw*>(a.rad) + eis * rw +
                                       rad_slot<L, M>(q0, lo, c0, a.C_n);
        // bf16: this lane's 16 channels of the radial slot, and below of each R
        // row, issued before the LDS round trips that transpose the block (one
        // memory latency per block rather than one per 4 channels); fp32 (twice
        // the registers) loads them where they are used
        constexpr bool PF = sizeof(typename TM::raw) == 2;
        uint4 rv_u[NU];
        if constexpr (PF) {
#pragma unroll
          for (int k = 0; k < NU; ++k) rv_u[k] = reinterpret_cast<const uint4*>(radp)[k];
        }
        float dr[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) dr[k] = 0.f;
        static_for<nqm>([&](auto QI) {
          constexpr int q = q0 + decltype(QI)::value;
          constexpr int slot = sb + P::qtype(q, lo);
          __builtin_amdgcn_sched_barrier(0);  // one block at a time (register pressure)
          uint4 rr_u[NU];
          if constexpr (PF) {
#pragma unroll
            for (int k = 0; k < NU; ++k) rr_u[k] = reinterpret_cast<const uint4*>(rsave + P::mrow(q, lo) * a.C_n)[k];
          }
          // accumulator layout -> row layout
#pragma unroll
          for (int i = 0; i < 16; ++i) tb[tsw(8 * (i >> 2) + 4 * h + (i & 3), co)] = acc[slot][i];
          wave_sync();
#pragma unroll
          for (int g = 0; g < NU; ++g) {  // VEC channels at a time
            float rr[VEC], rv[VEC];
            if constexpr (PF) {
              unpack_vec<TM, VEC>(rr_u[g], rr);
              unpack_vec<TM, VEC>(rv_u[g], rv);
            } else {
              unpack_vec<TM, VEC>(reinterpret_cast<const uint4*>(rsave + P::mrow(q, lo) * a.C_n)[g], rr);
              unpack_vec<TM, VEC>(reinterpret_cast<const uint4*>(radp)[g], rv);
            }
#pragma unroll
            for (int g4 = 0; g4 < VEC / 4; ++g4) {
              const int cc = VEC * g + 4 * g4;
              float4 t4 = *reinterpret_cast<const float4*>(tb + tsw(co, 16 * h + cc));
              dr[cc] = fmaf(t4.x, rr[4 * g4], dr[cc]);
              dr[cc + 1] = fmaf(t4.y, rr[4 * g4 + 1], dr[cc + 1]);
              dr[cc + 2] = fmaf(t4.z, rr[4 * g4 + 2], dr[cc + 2]);
              dr[cc + 3] = fmaf(t4.w, rr[4 * g4 + 3], dr[cc + 3]);
              t4.x *= rv[4 * g4]; t4.y *= rv[4 * g4 + 1]; t4.z *= rv[4 * g4 + 2]; t4.w *= rv[4 * g4 + 3];
              *reinterpret_cast<float4*>(tb + tsw(co, 16 * h + cc)) = t4;
            }
          }
          wave_sync();
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[slot][i] = tb[tsw(8 * (i >> 2) + 4 * h + (i & 3), co)];
          wave_sync();
        });
        if (a.drad != nullptr && ei >= 0) {
          typename TM::raw* dp = reinterpret_cast<typename TM::raw*>(a.drad) + ei * rw +
                                 rad_slot<L, M>(q0, lo, c0, a.C_n);
          float t[8];
#pragma unroll
          for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int k = 0; k < 8; ++k) t[k] = dr[8 * half + k];
            store_vec<TM, 8>(dp + 8 * half, t);
          }
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
                                                    const float* wsh, const Args& a, int cb,
                                                    float* buf, int lane, uint64_t endmask) {
    constexpr int n = 2 * lo + 1;
    constexpr int nq = P::nq(lo);
    constexpr int PB = P::pblk(lo);
    const int co = lane & 31, h = lane >> 5;
    const float* Wl = wsh + P::woff(lo);
    const uint64_t startmask = (endmask << 1) | 1ull;
    for (int p = 0; p <= lo; ++p) {
      const bool has_col = 2 * p + h < n;
      const int ow = a.ow > 0 ? a.ow : a.C_n;
      const int ocb = a.ow > 0 ? cb - a.cb0 : cb;
      const int64_t colo = static_cast<int64_t>(lo * lo + 2 * p + h) * ow + ocb * CB + co;
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
        // chunk rows in edge order: X[0..3], Y[0..3], X[4..7], Y[4..7].  The
        // chunk's segment starts, opaque per chunk: otherwise the compiler
        // hoists all 64 uniform selects out of the column loop and spills them.
        uint32_t sm = static_cast<uint32_t>(startmask >> (c * P::CH)) & 0xffffu;
        asm volatile("" : "+s"(sm));
        static_for<P::CH>([&](auto UI) {
          constexpr int u = decltype(UI)::value;
          constexpr int k = 4 * (u >> 3) + (u & 3);
          const float val = ((u >> 2) & 1) ? Y[k] : X[k];
          run = ((sm >> u) & 1u) ? val : run + val;
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

  template <int W, int KR, bool RAD>
  static __device__ __forceinline__ void body(Smem& s, const float* wsh, char* st0, char* st1, char* st2,
                                              const Args& a,
                                              int cb, int tid, int nvalid) {
    const int wave = tid >> 6, lane = tid & 63;
    f32x16 acc[P::MSLOT];
#pragma unroll
    for (int k = 0; k < P::MSLOT; ++k)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[k][i] = 0.f;

    const int nks = a.C_k / KC;
    const char* wp = a.wpack + static_cast<int64_t>(cb) * a.frags_per_cb * FRAG;
    AState st;
    a_init<W>(st, s, a, lane);
    frag_t bn[P::NBW];
    // ring prologue, in the issue order kstep expects: DMA of step 0, B of
    // step 0, DMA of step 1
    a_dma<W, 0>(st, st0, a, 0);
    b_load<W, 0>(bn, wp, 0, 0, lane);
    if constexpr (KR == 3) {
      if constexpr (L >= 1) a_dma<W, (L >= 1 ? 1 : 0)>(st, st1, a, 0);
    } else {
      a_dma<W, 0>(st, st1, a, 1);
    }
    int64_t foff = 0;
    static_for<L + 1>([&](auto LIc) {
      constexpr int LI = decltype(LIc)::value;
      kdegree<W, LI, KR>(acc, bn, st, st0, st1, st2, a, wp, foff, nks, lane);
      foff += static_cast<int64_t>(nks) * P::nbfrag(LI);
    });
    __syncthreads();  // all A reads done before the stages become epilogue staging

    // segment ends of the tile: bit e set if edge e closes its segment
    const int le = lane < TE ? lane : TE - 1, ln = le + 1 < TE ? le + 1 : le;
    const uint64_t endmask = __ballot(lane < nvalid && (lane == nvalid - 1 || s.seg[ln] != s.seg[le]));
    const int col = cb * CB + (lane & 31);
    if constexpr (P::GW) {
      // bias and pre-activation rows; the gate values through the stages (every
      // wave passes the three barriers); the activation; the stores
      float* tb = wave_staging(wave, st0, st1, st2);
      static_for<L + 1>([&](auto LO) {
        constexpr int lo = decltype(LO)::value;
        if constexpr (P::tab.owner[lo] == W) {
          add_bias<lo>(acc, a, col);
          if (a.gsave != nullptr) save_pre<lo>(acc, s, a, cb, tb, lane);
        }
      });
      gate_rows<W>(acc, s, a, cb, tb, lane);
      __syncthreads();  // staging reads done before the gate values overwrite it
      gate_out<W>(acc, st0, st1, st2, lane);
      __syncthreads();
      static_for<L + 1>([&](auto LO) {
        constexpr int lo = decltype(LO)::value;
        if constexpr (P::tab.owner[lo] == W) gate_act_gw<lo>(acc, st0, st1, st2, lane);
      });
      __syncthreads();  // gate values read before the stages are staging again
      static_for<L + 1>([&](auto LO) {
        constexpr int lo = decltype(LO)::value;
        if constexpr (P::tab.owner[lo] == W) {
          if constexpr (MODE == FWD_EDGE)
            save_pre<lo, true>(acc, s, a, cb, tb, lane);
          else
            rotate_sum<W, lo>(acc, s, wsh, a, cb, tb, lane, endmask);
        }
      });
      return;
    }
    static_for<L + 1>([&](auto LO) {
      constexpr int lo = decltype(LO)::value;
      if constexpr (P::tab.owner[lo] == W) {
        if constexpr (!P::BWD) {
          add_bias<lo>(acc, a, col);
          if constexpr (GATE) {
            if (a.gsave != nullptr)
              save_pre<lo>(acc, s, a, cb,
                           wave_staging(wave, st0, st1, st2), lane);
            gate_act<lo>(acc);
          }
        } else if constexpr (RAD)
          radial<lo>(acc, s, a, cb,
                     wave_staging(wave, st0, st1, st2), lane);
        if constexpr (MODE == BWD_EDGE)
          store_gate_bwd<lo>(acc, s, a, cb,
                             wave_staging(wave, st0, st1, st2), lane);
        else if constexpr (MODE == FWD_EDGE)
          save_pre<lo, true>(acc, s, a, cb,
                             wave_staging(wave, st0, st1, st2), lane);
        else
          rotate_sum<W, lo>(acc, s, wsh, a, cb,
                            wave_staging(wave, st0, st1, st2),
                            lane, endmask);
      }
    });
  }

  template <int KR, bool RAD>
  static __device__ __forceinline__ void run(const Args& a) {
    __shared__ Smem s;
    __shared__ alignas(16) char st0[SB];
    __shared__ alignas(16) char st1[SB];
    __shared__ alignas(16) char st2[SB];
    // Wigner rows of the tile: its own LDS object, so that the compiler can tell
    // its DMA apart from the accesses to s
    __shared__ alignas(16) float wsh[P::W16P * 4];
    const int tid = threadIdx.x, wave = tid >> 6;
    // XCD-aware mapping: consecutive workgroup ids go round-robin over the 8
    // XCDs.  The n_cb channel-block workgroups of one edge tile are the
    // consecutive workgroups of one XCD, so they run together and read the
    // tile's rows from that XCD's L2 (each XCD holds the weights of all blocks).
    const int64_t bid = blockIdx.x;
    const int64_t slot = bid >> 3;
    const int cb = a.cb0 + static_cast<int>(slot % a.n_cb);
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
    // Segments cut by the tile boundary go to the partials buffer: the tile's
    // first segment (slot 0) if it began in an earlier tile, its last one
    // (slot 1) if it continues into the next tile.
    const bool fp = (e0 > 0) && (a.seg[e0 - 1] == a.seg[e0]);
    const bool lp = (e0 + nvalid < a.E) && (a.seg[e0 + nvalid] == a.seg[e0 + nvalid - 1]);
    if (tid < TE) {
      float* dst = nullptr;
      const int64_t ow = a.ow > 0 ? a.ow : a.C_n;
      if (tid < nvalid) {
        const int sg = s.seg[tid];
        const bool first = sg == s.seg[0], last = sg == s.seg[nvalid - 1];
        if ((first && fp) || (last && lp))
          dst = a.part + (tile * 2 + (first ? 0 : 1)) * d * ow;
        else
          dst = a.out + static_cast<int64_t>(sg) * d * ow;
      }
      s.optr[tid] = dst;
    }
    // Wigner rows of the tile's edges (pair layout): DMA straight into LDS,
    // issued after every global load whose value the prologue waits for, so it
    // is in flight with the first K steps; the K loop's waits and barriers
    // complete it long before the epilogue reads it.  Chunk i = 64 (k NW + w) +
    // lane is instruction k of wave w; lanes past the tile read an in-bounds row
    // into the padding; rows of edges past the tile are never stored.
    // FWD_EDGE and BWD_EDGE do not rotate back: no rows.
    if constexpr (MODE != FWD_EDGE && MODE != BWD_EDGE) {
      constexpr int R4 = P::WS / 4;
      const float4* dk4 = reinterpret_cast<const float4*>(a.dk);
      const int wv = __builtin_amdgcn_readfirstlane(wave), lane = tid & 63;
      for (int k = 0; k < (P::W16P / 64 + NW - 1) / NW; ++k) {
        const int blk = k * NW + wv;  // uniform
        if (blk >= P::W16P / 64) break;
        const int i = blk * 64 + lane;
        const int e = i / R4 < TE ? i / R4 : TE - 1;
        const int ei = s.eid[e] >= 0 ? s.eid[e] : s.eid[0];
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_global_load_lds(dk4 + static_cast<int64_t>(ei) * R4 + (i - (i / R4) * R4),
                                         (lds_void*)(reinterpret_cast<char*>(wsh) + blk * 1024), 16, 0, 0);
#endif
      }
    }
    static_for<NW>([&](auto WI) {
      constexpr int w = decltype(WI)::value;
      if (wave == w) body<w, KR, RAD>(s, wsh, st0, st1, st2, a, cb, tid, nvalid);
    });
  }
};

// KR: (C_k / KC) % 3 if C_k / KC >= 2, else 3.
// RAD (input gradient only): a radial scale is given (its gradient is formed).
// MINB: resident workgroups per CU the register allocation targets.
template <int L, int M, bool GATE, int NW, int RT, class TM, int MODE, int KR, bool RAD, int MINB>
__global__ __launch_bounds__(NW * 64, MINB) void gemm_kernel(Args a) {
  Gemm<L, M, GATE, NW, RT, TM, MODE>::template run<KR, RAD>(a);
}

}  // namespace msg
}  // namespace maloq
