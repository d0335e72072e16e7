// Device-side building blocks for per-edge Wigner-D matrices (gfx950).
//
// Conventions (reference src/maloq/helm/common/rotation.py):
//   * Euler angles of an edge vector v (already in the e3nn y-z-x frame,
//     esen_osh.py:318): u = v / max(|v|, 1e-12) clamped to [-1, 1];
//     beta = acos(u_y), alpha = atan2(u_x, u_z), gamma = U(0,1) * 2*pi and the
//     triple fed to wigner_D is (-gamma, -beta, -alpha)       (rotation.py:68-83).
//   * X_l(t)[i][i] = cos((l-i) t), X_l(t)[i][2l-i] = sin((l-i) t) with the
//     diagonal taking precedence at i = l                        (rotation.py:204-225).
//   * D_l = X_l(a) J_l X_l(b) J_l X_l(c)                         (rotation.py:189-201).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace maloq {

// Philox4x32-10 (Salmon et al., SC'11, "Parallel random numbers: as easy as
// 1, 2, 3"): counter = (edge, edge >> 32, 0, 0), key = (seed, seed >> 32).
__device__ __forceinline__ float philox_uniform(uint64_t seed, uint64_t edge) {
  uint32_t c0 = static_cast<uint32_t>(edge), c1 = static_cast<uint32_t>(edge >> 32);
  uint32_t c2 = 0u, c3 = 0u;
  uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t m0 = 0xD2511F53u, m1 = 0xCD9E8D57u;
    uint32_t hi0 = __umulhi(m0, c0), lo0 = m0 * c0;
    uint32_t hi1 = __umulhi(m1, c2), lo1 = m1 * c2;
    uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return static_cast<float>(c0 >> 8) * (1.0f / 16777216.0f);
}

// Returns the (alpha, beta, gamma) triple consumed by wigner_D.
__device__ __forceinline__ void edge_euler(float vx, float vy, float vz, float u01, float* a,
                                           float* b, float* c) {
  float n = sqrtf(vx * vx + vy * vy + vz * vz);
  n = fmaxf(n, 1e-12f);
  float x = fminf(fmaxf(vx / n, -1.0f), 1.0f);
  float y = fminf(fmaxf(vy / n, -1.0f), 1.0f);
  float z = fminf(fmaxf(vz / n, -1.0f), 1.0f);
  float beta = acosf(y);
  float alpha = atan2f(x, z);
  float gamma = u01 * 6.283185307179586f;
  *a = -gamma;
  *b = -beta;
  *c = -alpha;
}

__host__ __device__ constexpr int jd_size(int L) {
  int s = 0;
  for (int l = 0; l <= L; ++l) s += (2 * l + 1) * (2 * l + 1);
  return s;
}
__host__ __device__ constexpr int jd_offset(int l) {
  int s = 0;
  for (int k = 0; k < l; ++k) s += (2 * k + 1) * (2 * k + 1);
  return s;
}

// sin and cos of m t, the product and the trigonometry in fp64 and then
// rounded: the fp32 product m t alone would carry an error of up to
// |m t| 2^-24, which frequency m turns into O(1e-6) errors of D at l >= 5.
// Every kernel that builds Wigner blocks uses this, so their blocks agree bit
// for bit.
__device__ __forceinline__ void sincos_m(int m, float t, float* s, float* c) {
  double sd, cd;
  sincos(static_cast<double>(m) * static_cast<double>(t), &sd, &cd);
  *s = static_cast<float>(sd);
  *c = static_cast<float>(cd);
}

// cos / sin of (l - i) * t from a table of cos(m t), sin(m t), m = 0..L.
__device__ __forceinline__ float xcos(const float* tc, int f) { return tc[f < 0 ? -f : f]; }
__device__ __forceinline__ float xsin(const float* ts, int f) {
  return f < 0 ? -ts[-f] : ts[f];
}

// Row k of M2 = X(b) J X(c) for block l (length 2l+1) into m2row.
// J points to J_l (row-major), cc/sc: cos/sin table of angle c, cb/sb: of b.
__device__ __forceinline__ void wigner_m2_row(int l, int k, const float* J, const float* cb,
                                              const float* sb, const float* cc, const float* sc,
                                              float* m2row) {
  const int n = 2 * l + 1;
  const int kk = 2 * l - k;
  for (int j = 0; j < n; ++j) {
    const int f = l - j;
    float m1k, m1kk;
    if (j == l) {
      m1k = J[k * n + j];
      m1kk = J[kk * n + j];
    } else {
      const float cj = xcos(cc, f), sj = xsin(sc, f);
      m1k = J[k * n + j] * cj - J[k * n + (2 * l - j)] * sj;
      m1kk = J[kk * n + j] * cj - J[kk * n + (2 * l - j)] * sj;
    }
    float v;
    if (k == l) {
      v = m1k;
    } else {
      const int fk = l - k;
      v = xcos(cb, fk) * m1k + xsin(sb, fk) * m1kk;
    }
    m2row[j] = v;
  }
}

// Row i of D_l = X(a) J M2 into drow, with M2 (row-major, n x n) given.
__device__ __forceinline__ void wigner_d_row(int l, int i, const float* J, const float* M2,
                                             const float* ca, const float* sa, float* drow) {
  const int n = 2 * l + 1;
  const int ii = 2 * l - i;
  const int fi = l - i;
  const float c = (i == l) ? 1.0f : xcos(ca, fi);
  const float s = (i == l) ? 0.0f : xsin(sa, fi);
  for (int j = 0; j < n; ++j) {
    float a = 0.f, b = 0.f;
    for (int k = 0; k < n; ++k) {
      const float m = M2[k * n + j];
      a = fmaf(J[i * n + k], m, a);
      b = fmaf(J[ii * n + k], m, b);
    }
    drow[j] = (i == l) ? a : c * a + s * b;
  }
}

}  // namespace maloq
