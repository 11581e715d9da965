// Batched randomized SVD + INT8 epilogue (gfx950), one workgroup per matrix.
//
// Replaces batched_randomized_svd (rsvd.py:74-157) and the quantising part
// of _compress_tensor (spectral_cache.py:321-407, 481-516).
//
// Per matrix M [rows <= 512][cols in {64,128}] (fp16, exact in fp32):
//   Z   <- Omega                                   (given, or Philox4x32-10)
//   Y   <- M Z ;  Y <- orth(Y)                      \  n_iter times:
//   Z   <- M^T Y ; Y <- M Z ; Y <- orth(Y)          /  same subspace as the
//                                                     reference's (M M^T)^q M Omega
//   Bp^T <- M^T Y                                   (Bp = Q^T M, r x cols)
//   eig(Bp Bp^T) = W diag(lambda) W^T               (fp64 parallel Jacobi)
//   S = sqrt(lambda), Vh_i = (Bp^T W)_i / S_i (normalised), coeffs = Q W S
//   INT8 per head / per row, basis fp16.
// orth() is CholeskyQR in fp64 (one pass between iterations, two passes for
// the final Q); columns whose Cholesky pivot vanishes are zeroed, so
// rank-deficient blocks (zeros, repeated rows) stay finite.
// Thread t owns rows t and t+256 of Y/Q in registers; Y, Bp^T, the Gram
// matrices and W live in LDS.
#include <math.h>

#include "sc_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kMaxRows = 512;

struct RsvdParams {
  int count, inner, rows, cols, rank, rank_v, r, r_v, n_iter, kp, kp_v, gran, coeff_major, basis_dmajor, m_dtype;
  const char* m;
  long m_so, m_si, m_sr;
  const float* omega;
  unsigned long long seed;
  int8_t* codes;
  long codes_so, codes_si;
  float* scales;
  long sc_so, sc_si;
  float* minmax;
  long mm_so, mm_si;
  float* vnorm;
  long vn_so, vn_si;
  h16* basis;
  long bs_so, bs_si;
  float* coeffs_out;
  float* svals_out;
  float* vh_out;
  float* omega_out;
  // tier mode
  int tier_mode;
  int B, Hkv, NB, TCAP, max_new;
  const int32_t* tail_pos;
  int32_t* counters;
  int32_t* block_start;
  ScTierDesc tier;
};

struct Job {
  const char* src;  // row 0 (generic) or ring base (tier)
  long row_stride;  // generic, in elements
  int dtype, esize;  // SC_DTYPE_* of the input and its byte size
  int ring_head, ring_cap;  // ring_cap > 0 -> ring addressing
  int k, r, kp, coeff_major, basis_dmajor;
  int8_t* codes;
  float* scales;
  float* minmax;
  float* vnorm;
  h16* basis;
  unsigned long long stream;
  long index;  // generic matrix index (debug outputs), -1 in tier mode
};

__device__ __forceinline__ const char* row_ptr(const Job& j, int t, int cols) {
  if (j.ring_cap > 0) return j.src + (long)((j.ring_head + t) % j.ring_cap) * cols * j.esize;
  return j.src + (long)t * j.row_stride * j.esize;
}

// Eight consecutive input elements as fp32 (exact for fp16/bf16/fp32).
__device__ __forceinline__ void load8(const char* p, int dtype, float (&a)[8]) {
  if (dtype == SC_DTYPE_F16) {
    const half8_t h = *reinterpret_cast<const half8_t*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = (float)h[i];
  } else if (dtype == SC_DTYPE_F32) {
    const float4 x = reinterpret_cast<const float4*>(p)[0], y = reinterpret_cast<const float4*>(p)[1];
    a[0] = x.x, a[1] = x.y, a[2] = x.z, a[3] = x.w, a[4] = y.x, a[5] = y.y, a[6] = y.z, a[7] = y.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = __uint_as_float(w[i] << 16);
      a[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

__device__ __forceinline__ float load1(const char* p, int dtype) {
  if (dtype == SC_DTYPE_F16) return (float)*reinterpret_cast<const h16*>(p);
  if (dtype == SC_DTYPE_F32) return *reinterpret_cast<const float*>(p);
  return __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
}

// ------------------------------------------------------------ Philox RNG
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint2 k) {
#pragma unroll
  for (int i = 0; i < 10; ++i) {
    const uint32_t lo0 = c.x * 0xD2511F53u, hi0 = __umulhi(c.x, 0xD2511F53u);
    const uint32_t lo1 = c.z * 0xCD9E8D57u, hi1 = __umulhi(c.z, 0xCD9E8D57u);
    c = make_uint4(hi1 ^ c.y ^ k.x, lo1, hi0 ^ c.w ^ k.y, lo0);
    k.x += 0x9E3779B9u;
    k.y += 0xBB67AE85u;
  }
  return c;
}

// Two standard normals for element pair e2 of stream `stream` (Box-Muller).
__device__ __forceinline__ float2 gauss2(unsigned long long seed, unsigned long long stream, uint32_t e2) {
  const uint4 o = philox4x32_10(make_uint4(e2, (uint32_t)stream, (uint32_t)(stream >> 32), 0x5bd1e995u),
                                make_uint2((uint32_t)seed, (uint32_t)(seed >> 32)));
  const float u1 = ((o.x >> 8) + 1u) * (1.0f / 16777216.0f);  // (0, 1]
  const float u2 = (o.y >> 8) * (1.0f / 16777216.0f);         // [0, 1)
  const float rad = sqrtf(-2.0f * logf(u1));
  float s, c;
  sincosf(6.2831853071795865f * u2, &s, &c);
  return make_float2(rad * c, rad * s);
}

// ------------------------------------------------------- block helpers
template <int RM>
struct Lds {
  float* Ys;     // [kMaxRows][RM]  Y / Q rows, later Vh [RM][cols]
  float* Zs;     // [128][RM]       Z / Bp^T
  double* Gs;    // [RM][RM]
  double* Ws;    // [RM][RM]        R^-1, then eigenvectors
  float* Wf;     // [RM][RM]        W[:, ord] * S for the coefficient product
  double* red;   // [128]
  int* ord;      // [RM]
  int* flag;     // [RM + 4]
};

template <int RM>
__device__ Lds<RM> carve(void* base) {
  Lds<RM> l;
  char* p = (char*)base;
  l.Gs = (double*)p;
  p += sizeof(double) * RM * RM;
  l.Ws = (double*)p;
  p += sizeof(double) * RM * RM;
  l.red = (double*)p;
  p += sizeof(double) * 128;
  l.Ys = (float*)p;
  p += sizeof(float) * kMaxRows * RM;
  l.Zs = (float*)p;
  p += sizeof(float) * 128 * RM;
  l.Wf = (float*)p;
  p += sizeof(float) * RM * RM;
  l.ord = (int*)p;
  p += sizeof(int) * RM;
  l.flag = (int*)p;
  return l;
}

template <int RM>
constexpr size_t lds_bytes() {
  return sizeof(double) * (2 * RM * RM + 128) + sizeof(float) * (kMaxRows * RM + 128 * RM + RM * RM) +
         sizeof(int) * (2 * RM + 4);
}

// y[c] = sum_d M[row][d] Zs[d][c]
template <int RM>
__device__ void gemm_rows(const Job& j, int rows, int cols, const float* Zs, float (&y0)[RM], float (&y1)[RM]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < RM; ++c) y0[c] = y1[c] = 0.f;
  const bool v0 = t < rows, v1 = t + kThreads < rows;
  const char* r0 = v0 ? row_ptr(j, t, cols) : nullptr;
  const char* r1 = v1 ? row_ptr(j, t + kThreads, cols) : nullptr;
  for (int d0 = 0; d0 < cols; d0 += 8) {
    float m0[8], m1[8];
    if (v0) load8(r0 + (long)d0 * j.esize, j.dtype, m0);
    else
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) m0[dd] = 0.f;
    if (v1) load8(r1 + (long)d0 * j.esize, j.dtype, m1);
    else
#pragma unroll
      for (int dd = 0; dd < 8; ++dd) m1[dd] = 0.f;
#pragma unroll
    for (int dd = 0; dd < 8; ++dd) {
      const float a0 = m0[dd], a1 = m1[dd];
      const float* z = Zs + (d0 + dd) * RM;
#pragma unroll
      for (int c = 0; c < RM; ++c) {
        const float zc = z[c];
        y0[c] = fmaf(a0, zc, y0[c]);
        y1[c] = fmaf(a1, zc, y1[c]);
      }
    }
  }
}

template <int RM>
__device__ void store_rows(float* Ys, int rows, const float (&y0)[RM], const float (&y1)[RM]) {
  const int t = threadIdx.x;
  if (t < rows)
#pragma unroll
    for (int c = 0; c < RM; ++c) Ys[t * RM + c] = y0[c];
  if (t + kThreads < rows)
#pragma unroll
    for (int c = 0; c < RM; ++c) Ys[(t + kThreads) * RM + c] = y1[c];
}

// Zs[d][c] = sum_row M[row][d] Ys[row][c]   (M^T Y)
template <int RM>
__device__ void gemm_cols(const Job& j, int rows, int cols, const float* Ys, float* Zs) {
  const int t = threadIdx.x;
  const int groups = kThreads / cols;  // 2 (cols 128) or 4 (cols 64)
  const int d = t % cols, cg = t / cols;
  constexpr int CW2 = RM / 2, CW4 = RM / 4;
  const int cw = groups == 2 ? CW2 : CW4;
  const int c0 = cg * cw;
  float z[CW2];
#pragma unroll
  for (int c = 0; c < CW2; ++c) z[c] = 0.f;
  for (int row = 0; row < rows; ++row) {
    const float mv = load1(row_ptr(j, row, cols) + (long)d * j.esize, j.dtype);
    const float* y = Ys + row * RM + c0;
#pragma unroll
    for (int c = 0; c < CW2; ++c)
      if (c < cw) z[c] = fmaf(mv, y[c], z[c]);
  }
#pragma unroll
  for (int c = 0; c < CW2; ++c)
    if (c < cw) Zs[d * RM + c0 + c] = z[c];
}

// Gs = A^T A (fp64) for A = S[nrows][RM] (first r columns).
template <int RM>
__device__ void gram(const float* S, int nrows, int r, double* Gs) {
  const int npairs = r * (r + 1) / 2;
  for (int pidx = threadIdx.x; pidx < npairs; pidx += kThreads) {
    int c1 = 0, rem = pidx;
    while (rem >= r - c1) {
      rem -= r - c1;
      ++c1;
    }
    const int c2 = c1 + rem;
    double acc = 0.0;
    for (int row = 0; row < nrows; ++row) acc = fma((double)S[row * RM + c1], (double)S[row * RM + c2], acc);
    Gs[c1 * RM + c2] = acc;
    Gs[c2 * RM + c1] = acc;
  }
}

// In-place Cholesky G = L L^T (lower part of Gs), then Ws = L^{-T} (upper
// triangular R^{-1} with R = L^T).  Vanishing pivots mark dead columns.
template <int RM>
__device__ void cholesky_rinv(double* Gs, double* Ws, int* dead, double* red, int r) {
  const int t = threadIdx.x;
  if (t == 0) {
    double gmax = 0.0;
    for (int c = 0; c < r; ++c) gmax = fmax(gmax, Gs[c * RM + c]);
    red[0] = gmax;
  }
  __syncthreads();
  const double tol = red[0] * 1e-26 + 1e-300;
  for (int jc = 0; jc < r; ++jc) {
    // column jc of L: pivot then scale
    const double piv = Gs[jc * RM + jc];
    const bool is_dead = !(piv > tol);
    const double lj = is_dead ? 1.0 : sqrt(piv);
    __syncthreads();
    for (int i = jc + 1 + t; i < r; i += kThreads) Gs[i * RM + jc] = is_dead ? 0.0 : Gs[i * RM + jc] / lj;
    if (t == 0) {
      Gs[jc * RM + jc] = lj;
      dead[jc] = is_dead;
    }
    __syncthreads();
    const int m = r - jc - 1;
    for (int e = t; e < m * m; e += kThreads) {
      const int i = jc + 1 + e / m, k = jc + 1 + e % m;
      if (k <= i) Gs[i * RM + k] -= Gs[i * RM + jc] * Gs[k * RM + jc];
    }
    __syncthreads();
  }
  // R = L^T upper.  Solve R X = I column by column (thread = column).
  if (t < r) {
    const int c = t;
    for (int i = r - 1; i >= 0; --i) {
      double v = (i == c) ? 1.0 : 0.0;
      for (int m2 = i + 1; m2 <= c; ++m2) v -= Gs[m2 * RM + i] * Ws[m2 * RM + c];  // R[i][m2] = L[m2][i]
      Ws[i * RM + c] = (i > c) ? 0.0 : v / Gs[i * RM + i];
    }
    if (dead[c])
      for (int i = 0; i < r; ++i) Ws[i * RM + c] = 0.0;
  }
  __syncthreads();
}

// y <- y R^{-1}
template <int RM>
__device__ void apply_rinv(const double* Ws, int r, float (&y0)[RM], float (&y1)[RM]) {
  float q0[RM], q1[RM];
#pragma unroll
  for (int c = 0; c < RM; ++c) {
    double a0 = 0.0, a1 = 0.0;
#pragma unroll
    for (int i = 0; i <= c; ++i) {
      const double w = Ws[i * RM + c];
      a0 = fma((double)y0[i], w, a0);
      a1 = fma((double)y1[i], w, a1);
    }
    q0[c] = c < r ? (float)a0 : 0.f;
    q1[c] = c < r ? (float)a1 : 0.f;
  }
#pragma unroll
  for (int c = 0; c < RM; ++c) {
    y0[c] = q0[c];
    y1[c] = q1[c];
  }
}

template <int RM>
__device__ void orth(Lds<RM>& L, int rows, int r, int passes, float (&y0)[RM], float (&y1)[RM]) {
  for (int ps = 0; ps < passes; ++ps) {
    __syncthreads();
    store_rows<RM>(L.Ys, rows, y0, y1);
    __syncthreads();
    gram<RM>(L.Ys, rows, r, L.Gs);
    __syncthreads();
    cholesky_rinv<RM>(L.Gs, L.Ws, L.flag, L.red, r);
    apply_rinv<RM>(L.Ws, r, y0, y1);
  }
}

// Cyclic parallel Jacobi on the symmetric Gs (r x r): Gs -> diag, Ws = V.
template <int RM>
__device__ void jacobi_eig(double* Gs, double* Ws, double* red, int* flag, int r) {
  const int t = threadIdx.x;
  for (int e = t; e < RM * RM; e += kThreads) Ws[e] = (e / RM == e % RM) ? 1.0 : 0.0;
  const int ne = r + (r & 1);  // even player count (player r is a bye when r odd)
  double* rot = red;           // [c, s, p, q] per pair, up to 20 pairs (80 doubles)
  __syncthreads();
  for (int sweep = 0; sweep < 30; ++sweep) {
    // convergence test: off-diagonal vs diagonal mass
    if (t == 0) {
      double off = 0.0, dia = 0.0;
      for (int i = 0; i < r; ++i)
        for (int k = 0; k < r; ++k) {
          const double v = Gs[i * RM + k];
          if (i == k)
            dia += v * v;
          else
            off += v * v;
        }
      flag[RM] = (off <= 1e-30 * dia) || (dia == 0.0);
    }
    __syncthreads();
    if (flag[RM]) break;
    for (int step = 0; step < ne - 1; ++step) {
      // round-robin pairing: player 0 fixed, others rotate
      if (t < ne / 2) {
        auto player = [&](int idx) { return idx == 0 ? 0 : 1 + (idx - 1 + step) % (ne - 1); };
        int p = player(t), q = player(ne - 1 - t);
        if (p > q) {
          const int tmp = p;
          p = q;
          q = tmp;
        }
        double c = 1.0, s = 0.0;
        if (q < r) {
          const double apq = Gs[p * RM + q];
          if (apq != 0.0) {
            const double app = Gs[p * RM + p], aqq = Gs[q * RM + q];
            const double tau = (aqq - app) / (2.0 * apq);
            const double tt = (tau >= 0.0 ? 1.0 : -1.0) / (fabs(tau) + sqrt(1.0 + tau * tau));
            c = 1.0 / sqrt(1.0 + tt * tt);
            s = tt * c;
          }
        }
        rot[4 * t] = c;
        rot[4 * t + 1] = s;
        rot[4 * t + 2] = p;
        rot[4 * t + 3] = q;
      }
      __syncthreads();
      // rows: A <- J^T A
      for (int e = t; e < (ne / 2) * r; e += kThreads) {
        const int pi = e / r, k = e % r;
        const double c = rot[4 * pi], s = rot[4 * pi + 1];
        const int p = (int)rot[4 * pi + 2], q = (int)rot[4 * pi + 3];
        if (q < r && s != 0.0) {
          const double ap = Gs[p * RM + k], aq = Gs[q * RM + k];
          Gs[p * RM + k] = c * ap - s * aq;
          Gs[q * RM + k] = s * ap + c * aq;
        }
      }
      __syncthreads();
      // columns: A <- A J, V <- V J
      for (int e = t; e < (ne / 2) * r; e += kThreads) {
        const int pi = e / r, k = e % r;
        const double c = rot[4 * pi], s = rot[4 * pi + 1];
        const int p = (int)rot[4 * pi + 2], q = (int)rot[4 * pi + 3];
        if (q < r && s != 0.0) {
          const double ap = Gs[k * RM + p], aq = Gs[k * RM + q];
          Gs[k * RM + p] = c * ap - s * aq;
          Gs[k * RM + q] = s * ap + c * aq;
          const double vp = Ws[k * RM + p], vq = Ws[k * RM + q];
          Ws[k * RM + p] = c * vp - s * vq;
          Ws[k * RM + q] = s * vp + c * vq;
        }
      }
      __syncthreads();
    }
  }
  __syncthreads();
}

template <int RM>
__device__ void run_matrix(const RsvdParams& p, const Job& j, int rows, int cols, int n_iter, Lds<RM>& L,
                           const float* omega_in, long dbg_index) {
  const int t = threadIdx.x;
  const int r = j.r, k = j.k;
  // ---- sketch
  for (int e = t; e < 128 * RM; e += kThreads) L.Zs[e] = 0.f;
  __syncthreads();
  if (omega_in) {
    for (int e = t; e < cols * r; e += kThreads) L.Zs[(e / r) * RM + e % r] = omega_in[e];
  } else {
    for (int e2 = t; e2 < (cols * r + 1) / 2; e2 += kThreads) {
      const float2 z = gauss2(p.seed, j.stream, (uint32_t)e2);
      const int e = 2 * e2;
      L.Zs[(e / r) * RM + e % r] = z.x;
      if (e + 1 < cols * r) L.Zs[((e + 1) / r) * RM + (e + 1) % r] = z.y;
    }
  }
  __syncthreads();
  if (p.omega_out && dbg_index >= 0)
    for (int e = t; e < cols * r; e += kThreads) p.omega_out[dbg_index * cols * r + e] = L.Zs[(e / r) * RM + e % r];

  float y0[RM], y1[RM];
  gemm_rows<RM>(j, rows, cols, L.Zs, y0, y1);
  orth<RM>(L, rows, r, 1, y0, y1);
  for (int it = 0; it < n_iter; ++it) {
    __syncthreads();
    store_rows<RM>(L.Ys, rows, y0, y1);
    __syncthreads();
    gemm_cols<RM>(j, rows, cols, L.Ys, L.Zs);
    __syncthreads();
    gemm_rows<RM>(j, rows, cols, L.Zs, y0, y1);
    orth<RM>(L, rows, r, it + 1 == n_iter ? 2 : 1, y0, y1);
  }
  if (n_iter == 0) orth<RM>(L, rows, r, 1, y0, y1);  // second pass for the final Q
  // ---- Bp^T = M^T Q
  __syncthreads();
  store_rows<RM>(L.Ys, rows, y0, y1);
  __syncthreads();
  gemm_cols<RM>(j, rows, cols, L.Ys, L.Zs);
  __syncthreads();
  gram<RM>(L.Zs, cols, r, L.Gs);  // Bp Bp^T
  __syncthreads();
  jacobi_eig<RM>(L.Gs, L.Ws, L.red, L.flag, r);
  // ---- sort eigenvalues (descending)
  if (t == 0) {
    for (int c = 0; c < r; ++c) L.ord[c] = c;
    for (int a = 0; a < r; ++a) {
      int best = a;
      for (int b2 = a + 1; b2 < r; ++b2)
        if (L.Gs[L.ord[b2] * RM + L.ord[b2]] > L.Gs[L.ord[best] * RM + L.ord[best]]) best = b2;
      const int tmp = L.ord[a];
      L.ord[a] = L.ord[best];
      L.ord[best] = tmp;
    }
  }
  __syncthreads();
  // Wf[c][i] = W[c][ord_i] * S_i  (i < k)
  for (int e = t; e < r * k; e += kThreads) {
    const int c = e / k, i = e % k;
    const int oi = L.ord[i];
    const double sv = sqrt(fmax(L.Gs[oi * RM + oi], 0.0));
    L.Wf[c * RM + i] = (float)(L.Ws[c * RM + oi] * sv);
  }
  // Vh (unnormalised) into Ys as [k][cols]: Vh_i[d] = sum_c W[c][ord_i] Bp^T[d][c]
  for (int e = t; e < k * cols; e += kThreads) {
    const int i = e / cols, d = e % cols;
    const int oi = L.ord[i];
    double acc = 0.0;
    for (int c = 0; c < r; ++c) acc = fma(L.Ws[c * RM + oi], (double)L.Zs[d * RM + c], acc);
    L.Ys[i * cols + d] = (float)acc;
  }
  __syncthreads();
  if (t < k) {  // row norms -> 1/norm (0 for vanished rows)
    double nn = 0.0;
    for (int d = 0; d < cols; ++d) {
      const double v = L.Ys[t * cols + d];
      nn += v * v;
    }
    L.red[t] = nn > 0.0 ? 1.0 / sqrt(nn) : 0.0;
    if (p.svals_out && dbg_index >= 0) {
      const int oi = L.ord[t];
      p.svals_out[dbg_index * k + t] = (float)sqrt(fmax(L.Gs[oi * RM + oi], 0.0));
    }
  }
  __syncthreads();
  // basis
  for (int e = t; e < j.kp * cols; e += kThreads) {
    const int i = e / cols, d = e % cols;
    const float v = i < k ? (float)(L.Ys[i * cols + d] * L.red[i]) : 0.f;
    if (j.basis_dmajor)
      j.basis[(long)d * j.kp + i] = (h16)v;
    else
      j.basis[(long)i * cols + d] = (h16)v;
    if (p.vh_out && dbg_index >= 0 && i < k) p.vh_out[(dbg_index * k + i) * cols + d] = v;
  }
  // ---- coefficients of my rows: coeff[i] = sum_c Q[row][c] Wf[c][i]
  float cf0[RM], cf1[RM];
#pragma unroll
  for (int i = 0; i < RM; ++i) {
    float a0 = 0.f, a1 = 0.f;
    if (i < k) {
#pragma unroll
      for (int c = 0; c < RM; ++c) {
        if (c < r) {
          const float w = L.Wf[c * RM + i];
          a0 = fmaf(y0[c], w, a0);
          a1 = fmaf(y1[c], w, a1);
        }
      }
    }
    cf0[i] = a0;
    cf1[i] = a1;
  }
  const bool v0 = t < rows, v1 = t + kThreads < rows;
  if (p.coeffs_out && dbg_index >= 0) {
    for (int i = 0; i < k; ++i) {
      if (v0) p.coeffs_out[(dbg_index * rows + t) * k + i] = cf0[i];
      if (v1) p.coeffs_out[(dbg_index * rows + t + kThreads) * k + i] = cf1[i];
    }
  }
  // ---- quantise (spectral_cache.py:481-516 formula)
  float am0 = 0.f, am1 = 0.f, mn = INFINITY, mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < RM; ++i)
    if (i < k) {
      if (v0) {
        am0 = fmaxf(am0, fabsf(cf0[i]));
        mn = fminf(mn, cf0[i]);
        mx = fmaxf(mx, cf0[i]);
      }
      if (v1) {
        am1 = fmaxf(am1, fabsf(cf1[i]));
        mn = fminf(mn, cf1[i]);
        mx = fmaxf(mx, cf1[i]);
      }
    }
  // block reductions: absmax, min, max
  float* fred = (float*)L.red;
  __syncthreads();
  {
    const float wa = wave_max(fmaxf(am0, am1)), wmn = -wave_max(-mn), wmx = wave_max(mx);
    if ((t & 63) == 0) {
      fred[t >> 6] = wa;
      fred[4 + (t >> 6)] = wmn;
      fred[8 + (t >> 6)] = wmx;
    }
  }
  __syncthreads();
  const float g_am = fmaxf(fmaxf(fred[0], fred[1]), fmaxf(fred[2], fred[3]));
  const float g_mn = fminf(fminf(fred[4], fred[5]), fminf(fred[6], fred[7]));
  const float g_mx = fmaxf(fmaxf(fred[8], fred[9]), fmaxf(fred[10], fred[11]));
  const bool per_row = p.gran == SC_QUANT_PER_ROW;
  const float sh = fmaxf(g_am, 1e-8f) / 127.0f;
  const float s0 = per_row ? fmaxf(am0, 1e-8f) / 127.0f : sh;
  const float s1 = per_row ? fmaxf(am1, 1e-8f) / 127.0f : sh;
  float smax = sh;
  if (per_row) {
    __syncthreads();
    const float ws = wave_max(fmaxf(v0 ? s0 : 0.f, v1 ? s1 : 0.f));
    if ((t & 63) == 0) fred[12 + (t >> 6)] = ws;
    __syncthreads();
    smax = fmaxf(fmaxf(fred[12], fred[13]), fmaxf(fred[14], fred[15]));
  }
  auto put = [&](int i, int8_t q0, int8_t q1) {
    if (j.coeff_major) {
      if (v0) j.codes[(long)i * rows + t] = q0;
      if (v1) j.codes[(long)i * rows + t + kThreads] = q1;
    } else {
      if (v0) j.codes[(long)t * j.kp + i] = q0;
      if (v1) j.codes[(long)(t + kThreads) * j.kp + i] = q1;
    }
  };
#pragma unroll
  for (int i = 0; i < RM; ++i) {
    if (i < j.kp) {
      int8_t q0 = 0, q1 = 0;
      if (i < k) {
        q0 = (int8_t)(int)rintf(cf0[i] / s0);  // IEEE division, ties to even
        q1 = (int8_t)(int)rintf(cf1[i] / s1);
      }
      put(i, q0, q1);
    }
  }
  for (int i = RM; i < j.kp; ++i) put(i, 0, 0);
  if (per_row) {
    if (v0) j.scales[t] = s0;
    if (v1) j.scales[t + kThreads] = s1;
  } else if (t == 0) {
    j.scales[0] = sh;
  }
  if (t == 0) {
    if (j.minmax) {
      j.minmax[0] = g_mn;
      j.minmax[1] = g_mx;
    }
    if (j.vnorm) {
      int e2;
      frexpf(smax, &e2);
      j.vnorm[0] = ldexpf(1.0f, -e2);
    }
  }
}

template <int RM>
__global__ __launch_bounds__(kThreads) void rsvd_generic_kernel(RsvdParams p) {
  extern __shared__ __align__(16) char smem[];
  Lds<RM> L = carve<RM>(smem);
  const long i = blockIdx.x;
  const long io = i / p.inner, ii = i % p.inner;
  Job j;
  j.dtype = p.m_dtype;
  j.esize = p.m_dtype == SC_DTYPE_F32 ? 4 : 2;
  j.src = p.m + (io * p.m_so + ii * p.m_si) * j.esize;
  j.row_stride = p.m_sr;
  j.ring_head = 0;
  j.ring_cap = 0;
  j.k = p.rank;
  j.r = p.r;
  j.kp = p.kp;
  j.coeff_major = p.coeff_major;
  j.basis_dmajor = p.basis_dmajor;
  j.codes = p.codes + io * p.codes_so + ii * p.codes_si;
  j.scales = p.scales + io * p.sc_so + ii * p.sc_si;
  j.minmax = p.minmax ? p.minmax + io * p.mm_so + ii * p.mm_si : nullptr;
  j.vnorm = p.vnorm ? p.vnorm + io * p.vn_so + ii * p.vn_si : nullptr;
  j.basis = p.basis + io * p.bs_so + ii * p.bs_si;
  j.stream = (unsigned long long)i;
  j.index = i;
  run_matrix<RM>(p, j, p.rows, p.cols, p.n_iter, L, p.omega ? p.omega + i * (long)p.cols * p.r : nullptr, i);
}

// Tier mode: unit = (b, i, h, kind); compresses block i of sequence b's
// tail (if full) into cold slot NCOLD + i.
__device__ __forceinline__ int tier_new_blocks(const RsvdParams& p, const int32_t* cnt) {
  const int full = cnt[SC_CNT_TAIL_LEN] / p.tier.block_size;
  return max(0, min(min(full, p.max_new), p.NB - cnt[SC_CNT_NCOLD]));
}

template <int RM>
__global__ __launch_bounds__(kThreads) void rsvd_tier_kernel(RsvdParams p) {
  extern __shared__ __align__(16) char smem[];
  const int u = blockIdx.x;
  const int kind = u & 1;
  const int h = (u >> 1) % p.Hkv;
  const int i = ((u >> 1) / p.Hkv) % p.max_new;
  const int b = ((u >> 1) / p.Hkv) / p.max_new;
  const int32_t* cnt = p.counters + b * SC_NCOUNTERS;
  if (i >= tier_new_blocks(p, cnt)) return;
  Lds<RM> L = carve<RM>(smem);
  const ScTierDesc& T = p.tier;
  const int TB = T.block_size, D = T.head_dim;
  const int slot = cnt[SC_CNT_NCOLD] + i;
  const int head = (cnt[SC_CNT_TAIL_HEAD] + i * TB) % p.TCAP;
  const long bh = (long)b * p.Hkv + h;
  const long bhs = bh * p.NB + slot;
  const bool per_row = T.granularity == SC_QUANT_PER_ROW;
  Job j;
  j.dtype = SC_DTYPE_F16;
  j.esize = 2;
  j.src = (const char*)((const h16*)(kind ? T.tail_v : T.tail_k) + bh * p.TCAP * D);
  j.row_stride = D;
  j.ring_head = head;
  j.ring_cap = p.TCAP;
  j.k = kind ? T.k_values : T.k_keys;
  j.r = kind ? p.r_v : p.r;
  j.kp = kind ? T.kp_values : T.kp_keys;
  j.coeff_major = kind;
  j.basis_dmajor = 1;  // both bases d-major [cols][kp]
  j.codes = (kind ? T.codes_v : T.codes_k) + bhs * TB * j.kp;
  j.scales = (kind ? T.scales_v : T.scales_k) + (per_row ? bhs * TB : bhs);
  j.minmax = (kind ? T.minmax_v : T.minmax_k) ? (kind ? T.minmax_v : T.minmax_k) + bhs * 2 : nullptr;
  j.vnorm = kind ? T.vnorm + bhs : nullptr;
  j.basis = (h16*)(kind ? T.basis_v : T.basis_k) + bhs * (long)D * j.kp;
  j.stream = ((((unsigned long long)b * p.NB + slot) * p.Hkv + h) << 1) | kind;
  j.index = -1;
  if (threadIdx.x == 0 && h == 0 && kind == 0) p.block_start[b * p.NB + slot] = p.tail_pos[(long)b * p.TCAP + head];
  run_matrix<RM>(p, j, TB, D, p.n_iter, L, nullptr, -1);
}

__global__ void tier_compress_finalize(RsvdParams p) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= p.B) return;
  int32_t* cnt = p.counters + b * SC_NCOUNTERS;
  const int nb = tier_new_blocks(p, cnt);
  if (nb == 0) return;
  const int TB = p.tier.block_size;
  cnt[SC_CNT_NCOLD] += nb;
  cnt[SC_CNT_TAIL_HEAD] = (cnt[SC_CNT_TAIL_HEAD] + nb * TB) % p.TCAP;
  cnt[SC_CNT_TAIL_LEN] -= nb * TB;
  cnt[SC_CNT_COMPRESSIONS] += nb;
}

int pick_rm(int r) { return r <= 24 ? 24 : (r <= 40 ? 40 : 0); }

template <int RM>
int set_lds_limit(const void* fn) {
  SC_HIP_TRY(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes<RM>()));
  return SC_OK;
}

}  // namespace

extern "C" int sc_rsvd_compress(const ScCompressArgs* a, void* stream) {
  if (!a) return sc_fail(SC_ERR_INVALID, "sc_rsvd_compress: null args");
  if (a->count < 0 || a->inner < 1) return sc_fail(SC_ERR_INVALID, "bad count/inner");
  if (a->count == 0) return SC_OK;
  if (a->rows < 64 || a->rows > kMaxRows || a->rows % 64)
    return sc_fail(SC_ERR_UNSUPPORTED, "rows %d unsupported (multiple of 64, <= 512)", a->rows);
  if (a->cols != 64 && a->cols != 128) return sc_fail(SC_ERR_UNSUPPORTED, "cols %d unsupported (64/128)", a->cols);
  if (a->rank < 1 || a->oversample < 0 || a->n_iter < 0) return sc_fail(SC_ERR_INVALID, "bad rank/oversample/n_iter");
  const int r = a->rank + a->oversample < a->cols ? a->rank + a->oversample : a->cols;
  if (r >= a->cols - 1)
    return sc_fail(SC_ERR_UNSUPPORTED, "rank %d + oversample reaches the full-SVD edge (rsvd.py:84-87)", a->rank);
  const int rm = pick_rm(r);
  if (!rm) return sc_fail(SC_ERR_UNSUPPORTED, "rank + oversample = %d > 40", r);
  if (a->kp < a->rank) return sc_fail(SC_ERR_INVALID, "kp %d < rank %d", a->kp, a->rank);
  if (!a->m || !a->codes || !a->scales || !a->basis) return sc_fail(SC_ERR_INVALID, "null pointer");
  if (a->m_dtype < SC_DTYPE_F16 || a->m_dtype > SC_DTYPE_BF16) return sc_fail(SC_ERR_INVALID, "bad m_dtype");
  const int epr = a->m_dtype == SC_DTYPE_F32 ? 4 : 8;  // elements per 16 bytes
  if (((uintptr_t)a->m & 15) || (a->m_stride_row % epr) || (a->m_stride_inner % epr) || (a->m_stride_outer % epr))
    return sc_fail(SC_ERR_INVALID, "input rows must be 16-byte aligned");
  RsvdParams p = {};
  p.count = a->count;
  p.inner = a->inner;
  p.rows = a->rows;
  p.cols = a->cols;
  p.rank = a->rank;
  p.r = r;
  p.n_iter = a->n_iter;
  p.kp = a->kp;
  p.gran = a->granularity;
  p.coeff_major = a->coeff_major;
  p.basis_dmajor = a->basis_dmajor;
  p.m_dtype = a->m_dtype;
  p.m = (const char*)a->m;
  p.m_so = a->m_stride_outer;
  p.m_si = a->m_stride_inner;
  p.m_sr = a->m_stride_row;
  p.omega = a->omega;
  p.seed = a->seed;
  p.codes = a->codes;
  p.codes_so = a->codes_stride_outer;
  p.codes_si = a->codes_stride_inner;
  p.scales = a->scales;
  p.sc_so = a->scales_stride_outer;
  p.sc_si = a->scales_stride_inner;
  p.minmax = a->minmax;
  p.mm_so = a->minmax_stride_outer;
  p.mm_si = a->minmax_stride_inner;
  p.vnorm = a->vnorm;
  p.vn_so = a->vnorm_stride_outer;
  p.vn_si = a->vnorm_stride_inner;
  p.basis = (h16*)a->basis;
  p.bs_so = a->basis_stride_outer;
  p.bs_si = a->basis_stride_inner;
  p.coeffs_out = a->coeffs_out;
  p.svals_out = a->svals_out;
  p.vh_out = a->vh_out;
  p.omega_out = a->omega_out;
  hipStream_t s = (hipStream_t)stream;
  int rc;
  if (rm == 24) {
    if ((rc = set_lds_limit<24>((const void*)rsvd_generic_kernel<24>))) return rc;
    hipLaunchKernelGGL(rsvd_generic_kernel<24>, dim3(a->count), dim3(kThreads), lds_bytes<24>(), s, p);
  } else {
    if ((rc = set_lds_limit<40>((const void*)rsvd_generic_kernel<40>))) return rc;
    hipLaunchKernelGGL(rsvd_generic_kernel<40>, dim3(a->count), dim3(kThreads), lds_bytes<40>(), s, p);
  }
  return sc_launch_status("rsvd_generic_kernel");
}

extern "C" int sc_tier_compress(const ScTierDesc* t, int32_t max_new_blocks, int32_t n_iter, int32_t oversample,
                                uint64_t seed, void* stream) {
  if (!t || !t->counters) return sc_fail(SC_ERR_INVALID, "sc_tier_compress: null tier");
  if (max_new_blocks <= 0) return SC_OK;
  if (t->block_size < 64 || t->block_size > kMaxRows || t->block_size % 64)
    return sc_fail(SC_ERR_UNSUPPORTED, "block_size %d unsupported for compression", t->block_size);
  if (t->head_dim != 64 && t->head_dim != 128) return sc_fail(SC_ERR_UNSUPPORTED, "head_dim %d", t->head_dim);
  if (t->tail_capacity < t->block_size) return sc_fail(SC_ERR_INVALID, "tail capacity < block size");
  const int rk = t->k_keys + oversample < t->head_dim ? t->k_keys + oversample : t->head_dim;
  const int rv = t->k_values + oversample < t->head_dim ? t->k_values + oversample : t->head_dim;
  if (rk >= t->head_dim - 1 || rv >= t->head_dim - 1)
    return sc_fail(SC_ERR_UNSUPPORTED, "ranks reach the full-SVD edge (rsvd.py:84-87)");
  const int rm = pick_rm(rk > rv ? rk : rv);
  if (!rm) return sc_fail(SC_ERR_UNSUPPORTED, "rank + oversample > 40");
  if (t->kp_keys < t->k_keys || t->kp_values < t->k_values) return sc_fail(SC_ERR_INVALID, "kp < k");
  RsvdParams p = {};
  p.tier_mode = 1;
  p.tier = *t;
  p.B = t->batch;
  p.Hkv = t->kv_heads;
  p.NB = t->max_blocks;
  p.TCAP = t->tail_capacity;
  p.max_new = max_new_blocks;
  p.r = rk;
  p.r_v = rv;
  p.n_iter = n_iter;
  p.gran = t->granularity;
  p.seed = seed;
  p.tail_pos = t->tail_pos;
  p.counters = t->counters;
  p.block_start = t->block_start;
  hipStream_t s = (hipStream_t)stream;
  const int units = t->batch * max_new_blocks * t->kv_heads * 2;
  int rc;
  if (rm == 24) {
    if ((rc = set_lds_limit<24>((const void*)rsvd_tier_kernel<24>))) return rc;
    hipLaunchKernelGGL(rsvd_tier_kernel<24>, dim3(units), dim3(kThreads), lds_bytes<24>(), s, p);
  } else {
    if ((rc = set_lds_limit<40>((const void*)rsvd_tier_kernel<40>))) return rc;
    hipLaunchKernelGGL(rsvd_tier_kernel<40>, dim3(units), dim3(kThreads), lds_bytes<40>(), s, p);
  }
  if ((rc = sc_launch_status("rsvd_tier_kernel"))) return rc;
  hipLaunchKernelGGL(tier_compress_finalize, dim3((t->batch + 63) / 64), dim3(64), 0, s, p);
  return sc_launch_status("tier_compress_finalize");
}
