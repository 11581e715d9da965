// Batched randomized SVD + INT8 epilogue (gfx950), one workgroup per matrix.
//
// Replaces batched_randomized_svd (rsvd.py:74-157) and the quantising part
// of _compress_tensor (spectral_cache.py:321-407, 481-516).
//
// Per matrix M [rows <= 512][cols in {64,128}] (fp16/bf16/fp32, exact in fp32):
//   Z   <- Omega                                   (given, or Philox4x32-10)
//   Y   <- M Z, columns scaled to unit norm         (n_iter = 0: Y <- orth(Y), two passes)
//   Z   <- M^T Y ; Y <- M Z ; Y <- orth(Y)          n_iter times: same subspace as the
//                                                     reference's (M M^T)^q M Omega
//   Bp^T <- M^T Y                                   (Bp = Q^T M, r x cols)
//   eig(Bp Bp^T) = W diag(lambda) W^T               (fp64 parallel Jacobi)
//   S = sqrt(lambda), Vh_i = (Bp^T W)_i / S_i (normalised), coeffs = Q W S
//   INT8 per head / per row, basis fp16.
// Y, Z, Bp^T, the Gram matrices and W live in LDS.  For fp16 input the
// products with M run on MFMA (16x16x32 f16, the fp32 factor split into fp16
// hi + lo parts, so the result keeps fp32 accuracy) and the Gram matrices on
// the fp64 MFMA; other input types use fp32 VALU products.  orth() is
// CholeskyQR (one pass between iterations, two for the final Q): fp64
// Cholesky by one wave with its rows in registers, R^{-1} by all four waves,
// then Y <- Y R^{-1} row by row in fp32.  Columns whose Cholesky pivot
// vanishes are zeroed, so rank-deficient blocks (zeros, repeated rows) stay
// finite.
#include <math.h>

#include <utility>

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
  const float* row_weights;
  long rw_so, rw_si;
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
  const float* rw;  // row importances a[rows] (weighted compression) or nullptr
  float rw_mean;    // mean(a)
};

// Row weight of attention-weighted compression, sqrt(a / mean(a)) with IEEE
// division and square root (spectral_cache.py:356-358).
__device__ __forceinline__ float row_weight(const Job& j, int row) { return sqrtf(j.rw[row] / j.rw_mean); }

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
// p as an opaque LDS address: the accesses of a function then share one base
// register plus immediate offsets.  Without it the compiler folds every
// constant element offset into the array's constant address, and where that
// lies beyond the 64 KB reach of the immediate offset it keeps one address
// register per element, which spills.
template <class T>
__device__ __forceinline__ T* lds_base(T* p) {
  auto q = (__attribute__((address_space(3))) T*)p;
  asm volatile("" : "+v"(q));
  return (T*)q;
}

template <int RM>
struct Lds {
  float* Ys;     // [kMaxRows][RM]  Y / Q rows, later the coefficient rows
  float* Zs;     // [128][RM]       Z / Bp^T, later Vh [RM][cols]
  double* Gs;    // [RM][RM] + spare<RM>()
  double* G2;    // [RM][RM] + spare<RM>()  second buffer of the Jacobi iteration
  double* Ws;    // [RM][RM] + spare<RM>()  eigenvectors
  float* Wf;     // [RM][RM]        W[:, ord] * S for the coefficient product
  double* red;   // [128]
  int* ord;      // [RM]
  int* flag;     // [RM + 4]
};

// Spare doubles after each of Gs, G2 and Ws at RM = 40: per-lane sinks of
// the Jacobi rounds' unused stores (so that every store is unconditional).
// None at RM = 24, whose rounds mask the unused lanes instead: there the
// spares would push the later arrays past the 64 KB reach of an LDS
// instruction's immediate offset.
template <int RM>
constexpr int spare() {
  return RM > 24 ? 64 : 0;
}

template <int RM>
__device__ Lds<RM> carve(void* base) {
  Lds<RM> l;
  char* p = (char*)base;
  l.Gs = (double*)p;
  p += sizeof(double) * (RM * RM + spare<RM>());
  l.G2 = (double*)p;
  p += sizeof(double) * (RM * RM + spare<RM>());
  l.Ws = (double*)p;
  p += sizeof(double) * (RM * RM + spare<RM>());
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
  return sizeof(double) * (3 * (RM * RM + spare<RM>()) + 128) + sizeof(float) * (kMaxRows * RM + 128 * RM + RM * RM) +
         sizeof(int) * (2 * RM + 4);
}

// y[c] = sum_d M[row][d] Zs[d][c]
template <int RM>
__device__ __forceinline__ void gemm_rows(const Job& j, int rows, int cols, const float* Zs, float (&y0)[RM], float (&y1)[RM]) {
  const int t = threadIdx.x;
#pragma unroll
  for (int c = 0; c < RM; ++c) y0[c] = y1[c] = 0.f;
  const bool v0 = t < rows, v1 = t + kThreads < rows;
  const char* r0 = v0 ? row_ptr(j, t, cols) : nullptr;
  const char* r1 = v1 ? row_ptr(j, t + kThreads, cols) : nullptr;
  // weighted rows: (w M)[row][d] rounded to fp32 once, as X * W (spectral_cache.py:361-362)
  const float w0 = j.rw && v0 ? row_weight(j, t) : 1.f, w1 = j.rw && v1 ? row_weight(j, t + kThreads) : 1.f;
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
      const float a0 = m0[dd] * w0, a1 = m1[dd] * w1;
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
__device__ __forceinline__ void store_rows(float* Ys, int rows, const float (&y0)[RM], const float (&y1)[RM]) {
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
__device__ __forceinline__ void gemm_cols(const Job& j, int rows, int cols, const float* Ys, float* Zs) {
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
    float mv = load1(row_ptr(j, row, cols) + (long)d * j.esize, j.dtype);
    if (j.rw) mv *= row_weight(j, row);
    const float* y = Ys + row * RM + c0;
#pragma unroll
    for (int c = 0; c < CW2; ++c)
      if (c < cw) z[c] = fmaf(mv, y[c], z[c]);
  }
#pragma unroll
  for (int c = 0; c < CW2; ++c)
    if (c < cw) Zs[d * RM + c0 + c] = z[c];
}

// ------------------------------------------------ MFMA paths (fp16 input)
// Products with the fp16 matrix M run on MFMA with M exact and the fp32
// factor split into fp16 hi + lo parts (two MFMAs, fp32 accumulation): the
// result keeps fp32 accuracy.  Gram matrices use the fp64 MFMA.
typedef double double4_t __attribute__((ext_vector_type(4)));

// Eight fp32 values split into fp16 hi = (h16)v and lo = (h16)(v - hi),
// converted in pairs (packed fp32 -> fp16 conversions; the subtraction stays
// scalar fp32).
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void split16x8(const float (&v)[8], half8_t& hi, half8_t& lo) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const f32x2_t x = {v[e], v[e + 1]};
    const f16x2_t h = __builtin_convertvector(x, f16x2_t);
    const f32x2_t hb = __builtin_convertvector(h, f32x2_t);
    const f32x2_t r = {x.x - hb.x, x.y - hb.y};
    const f16x2_t l = __builtin_convertvector(r, f16x2_t);
    hi[e] = h.x;
    hi[e + 1] = h.y;
    lo[e] = l.x;
    lo[e + 1] = l.y;
  }
}

// One batch of a wave's row tiles of a 512x128 block for gemm_rows_mfma:
// tiles w + 4 (b0 + i), i < kRowBatch, as MFMA A operands.
constexpr int kRowBatch = 4;
struct RowBatch {
  half8_t a[kRowBatch][4];
};
__device__ __forceinline__ void load_row_batch(const Job& j, int b0, RowBatch& rb) {
  constexpr int NW = kThreads / 64;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15, w = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < kRowBatch; ++i) {
    const h16* rp = reinterpret_cast<const h16*>(row_ptr(j, 16 * (w + NW * (b0 + i)) + n, 128));
#pragma unroll
    for (int s = 0; s < 4; ++s) rb.a[i][s] = *reinterpret_cast<const half8_t*>(rp + 32 * s + 8 * g);
  }
}

// Ys[rows][RM] = M[rows][cols] Zs[cols][RM]; wave w takes row tiles w, w+4, ...
template <int RM>
__device__ __forceinline__ void gemm_rows_mfma(const Job& j, int rows, int cols, const float* Zs, float* Ys,
                                               const RowBatch* pre = nullptr) {
  Zs = lds_base(Zs);
  Ys = lds_base(Ys);
  constexpr int CT = (RM + 15) / 16;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15, w = threadIdx.x >> 6;
  const int KS = cols / 32;
  half8_t bh[4][CT], bl[4][CT];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c = 16 * ct + n;
      const bool in = s < KS && c < RM;  // s < KS is wave-uniform
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {  // clamped (in-bounds) loads and a select: no exec-masked loads
        const float z = Zs[(32 * min(s, KS - 1) + 8 * g + e) * RM + min(c, RM - 1)];
        v[e] = in ? z : 0.f;
      }
      split16x8(v, bh[s][ct], bl[s][ct]);
    }
  if (rows == kMaxRows && cols == 128) {
    // the block geometry: a wave's 8 row tiles in two batches of 4, each
    // batch's loads issued together (two memory round trips, not eight);
    // `pre` (when given) is the first batch, loaded by the caller earlier
    constexpr int NW = kThreads / 64, BT = kRowBatch;
    auto batch = [&](int b0, const RowBatch& rb) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < BT; ++i) {
        const int rt = w + NW * (b0 + i);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          float4_t acc = (float4_t)0.f;
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(rb.a[i][s], bh[s][ct], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(rb.a[i][s], bl[s][ct], acc, 0, 0, 0);
          }
          const int c = 16 * ct + n;
          if (c < RM)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) Ys[(16 * rt + 4 * g + jj) * RM + c] = acc[jj];
        }
      }
    };
    int b0 = 0;
    if (pre) {
      batch(0, *pre);
      b0 = BT;
    }
#pragma unroll 1
    for (; b0 < kMaxRows / 16 / NW; b0 += BT) {
      RowBatch rb;
      load_row_batch(j, b0, rb);
      batch(b0, rb);
    }
    return;
  }
  for (int rt = w; rt < rows / 16; rt += kThreads / 64) {
    const h16* rp = reinterpret_cast<const h16*>(row_ptr(j, 16 * rt + n, cols));
    half8_t a[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      a[s] = s < KS ? *reinterpret_cast<const half8_t*>(rp + 32 * s + 8 * g) : (half8_t)(h16)0;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float4_t acc = (float4_t)0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s)
        if (s < KS) {
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], bh[s][ct], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], bl[s][ct], acc, 0, 0, 0);
        }
      const int c = 16 * ct + n;
      if (c < RM)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) Ys[(16 * rt + 4 * g + jj) * RM + c] = acc[jj];
    }
  }
}

typedef short short4_t __attribute__((ext_vector_type(4)));
constexpr int kColTile = 32;  // rows of M staged per step of gemm_cols_mfma

// fp16 elements of gemm_cols_mfma's staging tile: 32 rows, padded by 8
// elements (16 bytes) so the transposing reads of 4 consecutive rows fall
// in distinct banks.
__host__ __device__ constexpr int col_stage_elems(int cols) { return kColTile * (cols + 8); }

// Zs[cols][RM] = M^T Ys for fp16 M.  M's rows are staged 32 at a time in
// LDS (`stage`, row-major) with 16-byte loads; the next 32 rows are held in
// registers while the current ones are consumed.  Lane (g, n)'s A operand
// is rows 8g .. 8g+7 of column 16 d + n, read by two ds_read_b64_tr_b16:
// that read gives lane j of a 16-lane group element j & 3 of the 4-element
// chunk addressed by lane 4e + (j >> 2), so lane L addresses row
// 8g + (L >> 2) (+4), columns 16 d + 4 (L & 3) .. +3.  Wave w owns d tiles
// w*DT .. w*DT+DT-1 (cols/16/4 each).
template <int RM>
__device__ __forceinline__ void gemm_cols_mfma(const Job& j, int rows, int cols, const float* Ys, float* Zs,
                                               h16* stage) {
  constexpr int CT = (RM + 15) / 16;
  static_assert(2 * RM * RM * sizeof(double) >= col_stage_elems(128) * sizeof(h16),
                "the staging tile fits the Gs + Ws region, which is dead while this runs");
  const int t = threadIdx.x, lane = t & 63, g = lane >> 4, n = lane & 15, w = t >> 6;
  const int DT = cols / 64;  // d tiles per wave: 2 (cols 128) or 1 (cols 64)
  const int pitch = cols + 8;
  const int cpr = cols / 8;  // 16-byte chunks per row
  const int nchunks = kColTile * cpr;  // 512 or 256: one or two per thread
  float4_t acc[2][CT];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[dt][ct] = (float4_t)0.f;
  // this thread's chunks t and t + kThreads of a tile: row c / cpr, 16-byte chunk c % cpr
  const int c0 = t, c1 = t + kThreads;
  const bool has1 = c1 < nchunks;
  uint4 nx0, nx1;
  auto fetch = [&](int k0) __attribute__((always_inline)) {
    nx0 = *reinterpret_cast<const uint4*>(row_ptr(j, k0 + c0 / cpr, cols) + (c0 % cpr) * 16);
    if (has1) nx1 = *reinterpret_cast<const uint4*>(row_ptr(j, k0 + c1 / cpr, cols) + (c1 % cpr) * 16);
  };
  auto put = [&]() __attribute__((always_inline)) {
    *reinterpret_cast<uint4*>(stage + (c0 / cpr) * pitch + (c0 % cpr) * 8) = nx0;
    if (has1) *reinterpret_cast<uint4*>(stage + (c1 / cpr) * pitch + (c1 % cpr) * 8) = nx1;
  };
  fetch(0);
  put();
  __syncthreads();
  for (int k0 = 0; k0 < rows; k0 += kColTile) {
    const bool more = k0 + kColTile < rows;
    if (more) fetch(k0 + kColTile);
    half8_t a[2];
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      if (dt < DT) {
        const h16* p0 = stage + (8 * g + (n >> 2)) * pitch + (w * DT + dt) * 16 + 4 * (n & 3);
        typedef __attribute__((address_space(3))) short4_t lds_s4;
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0));
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0 + 4 * pitch));
        const half4_t l4 = __builtin_bit_cast(half4_t, lo), h4 = __builtin_bit_cast(half4_t, hi);
        a[dt] = (half8_t){l4.x, l4.y, l4.z, l4.w, h4.x, h4.y, h4.z, h4.w};
      } else {
        a[dt] = (half8_t)(h16)0;
      }
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      const int c = 16 * ct + n;
      half8_t bh, bl;
      float yv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = Ys[(k0 + 8 * g + e) * RM + min(c, RM - 1)];  // in bounds: no exec branch
        yv[e] = c < RM ? y : 0.f;
      }
      split16x8(yv, bh, bl);
#pragma unroll
      for (int dt = 0; dt < 2; ++dt)
        if (dt < DT) {
          acc[dt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[dt], bh, acc[dt][ct], 0, 0, 0);
          acc[dt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[dt], bl, acc[dt][ct], 0, 0, 0);
        }
    }
    __syncthreads();  // every wave is done with this tile
    if (more) {
      put();
      __syncthreads();
    }
  }
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
    if (dt < DT)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int c = 16 * ct + n;
        if (c < RM)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) Zs[((w * DT + dt) * 16 + 4 * g + jj) * RM + c] = acc[dt][ct][jj];
      }
}

// gemm_cols_mfma for 128 columns of M with each wave on one column tile
// of Ys, so a wave splits one column tile into fp16 hi + lo per staged tile
// instead of all of them: two tiles (RM <= 32): wave w takes tile w & 1 and
// the four d tiles 4 (w >> 1) .. + 3; three tiles (RM <= 48): wave w < 3
// takes tile w and all eight d tiles, wave 3 only stages.  Staging as
// gemm_cols_mfma.
template <int RM>
__device__ __forceinline__ void gemm_cols_mfma_ct(const Job& j, int rows, const float* Ys, float* Zs, h16* stage) {
  Ys = lds_base(Ys);
  Zs = lds_base(Zs);
  // two staging buffers: `stage` and the output Zs, which is written only
  // after the last tile
  static_assert(sizeof(float) * 128 * RM >= sizeof(h16) * kColTile * (128 + 8), "a staged tile fits in Zs");
  h16* const stg[2] = {lds_base(stage), lds_base(reinterpret_cast<h16*>(Zs))};
  constexpr int CT = (RM + 15) / 16;
  static_assert(CT == 2 || CT == 3, "two or three column tiles of Ys");
  constexpr int NDT = CT == 2 ? 4 : 8;  // d tiles per wave
  constexpr int cols = 128, pitch = cols + 8, cpr = cols / 8;
  static_assert(kColTile * cpr == 2 * kThreads, "two 16-byte chunks per thread and tile");
  const int t = threadIdx.x, lane = t & 63, g = lane >> 4, n = lane & 15, w = t >> 6;
  const int ct = CT == 2 ? (w & 1) : w, dt0 = CT == 2 ? 4 * (w >> 1) : 0;
  const bool busy = ct < CT;  // wave-uniform
  const int c = 16 * ct + n;
  float4_t acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = (float4_t)0.f;
  const int c0 = t, c1 = t + kThreads;
  // up to two tiles of M in flight in registers beyond the staged one
  uint4 nx0, nx1, nn0, nn1;
  auto fetch = [&](int k0, uint4& x0, uint4& x1) __attribute__((always_inline)) {
    x0 = *reinterpret_cast<const uint4*>(row_ptr(j, k0 + c0 / cpr, cols) + (c0 % cpr) * 16);
    x1 = *reinterpret_cast<const uint4*>(row_ptr(j, k0 + c1 / cpr, cols) + (c1 % cpr) * 16);
  };
  auto put = [&](h16* stage, const uint4& x0, const uint4& x1) __attribute__((always_inline)) {
    *reinterpret_cast<uint4*>(stage + (c0 / cpr) * pitch + (c0 % cpr) * 8) = x0;
    *reinterpret_cast<uint4*>(stage + (c1 / cpr) * pitch + (c1 % cpr) * 8) = x1;
  };
  fetch(0, nx0, nx1);
  if (kColTile < rows) fetch(kColTile, nn0, nn1);
  put(stg[0], nx0, nx1);
  __syncthreads();
  // step(k0, a, b) with tile k0 staged in stg[sb]: b holds tile k0 +
  // kColTile (in flight), a is free and receives tile k0 + 2 kColTile.
  // After the tile's products, b goes to the other buffer (last read by the
  // previous tile, before the barrier that ended it): one barrier per tile.
  // Two steps per iteration swap the register roles (no register copies,
  // which would wait for the loads).
  auto step = [&](int k0, int sb, uint4& a0, uint4& a1, const uint4& b0, const uint4& b1) __attribute__((always_inline)) {
    const h16* stage = stg[sb];
    if (k0 + 2 * kColTile < rows) fetch(k0 + 2 * kColTile, a0, a1);
    if (busy) {
      half8_t a[NDT];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const h16* p0 = stage + (8 * g + (n >> 2)) * pitch + (dt0 + dt) * 16 + 4 * (n & 3);
        typedef __attribute__((address_space(3))) short4_t lds_s4;
        const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0));
        const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0 + 4 * pitch));
        const half4_t l4 = __builtin_bit_cast(half4_t, lo), h4 = __builtin_bit_cast(half4_t, hi);
        a[dt] = (half8_t){l4.x, l4.y, l4.z, l4.w, h4.x, h4.y, h4.z, h4.w};
      }
      float yv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = Ys[(k0 + 8 * g + e) * RM + min(c, RM - 1)];  // in bounds: no exec branch
        yv[e] = c < RM ? y : 0.f;
      }
      half8_t bh, bl;
      split16x8(yv, bh, bl);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[dt], bh, acc[dt], 0, 0, 0);
        acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[dt], bl, acc[dt], 0, 0, 0);
      }
    }
    if (k0 + kColTile < rows) put(stg[sb ^ 1], b0, b1);
    __syncthreads();  // this tile's reads and the next tile's stores are done
  };
  for (int k0 = 0; k0 < rows; k0 += 2 * kColTile) {
    step(k0, 0, nx0, nx1, nn0, nn1);
    if (k0 + kColTile < rows) step(k0 + kColTile, 1, nn0, nn1, nx0, nx1);
  }
  if (busy && c < RM)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) Zs[((dt0 + dt) * 16 + 4 * g + jj) * RM + c] = acc[dt][jj];
}

// Gs[c1][c2] = sum_row S[row][c1] S[row][c2] (c1, c2 < r) in fp64 on MFMA
// (nrows a multiple of 16).
// Tile (ta, tb), ta <= tb, of the CT x CT upper triangle goes to wave
// (tile index) % 4; the f64 16x16x4 output holds D[4 e + g][n] in lane
// (g, n), element e.
template <int RM>
__device__ __forceinline__ void gram_mfma(const float* S, int nrows, int r, double* Gs) {
  S = lds_base(S);
  Gs = lds_base(Gs);
  constexpr int CT = (RM + 15) / 16;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15, w = threadIdx.x >> 6;
  int tix = 0;
  for (int ta = 0; ta < CT; ++ta)
    for (int tb = ta; tb < CT; ++tb, ++tix) {
      if (tix % (kThreads / 64) != w) continue;
      const int ca = 16 * ta + n, cb = 16 * tb + n;
      // four independent accumulation chains (rows k0 + 4u + g), summed in
      // a fixed order at the end
      double4_t acc = {0.0, 0.0, 0.0, 0.0}, acc1 = acc, acc2 = acc, acc3 = acc;
      auto step = [&](int k0) __attribute__((always_inline)) {
        double av[4], bv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float sa = S[(k0 + 4 * u + g) * RM + min(ca, RM - 1)], sb = S[(k0 + 4 * u + g) * RM + min(cb, RM - 1)];
          av[u] = ca < RM ? (double)sa : 0.0;
          bv[u] = cb < RM ? (double)sb : 0.0;
        }
        acc = __builtin_amdgcn_mfma_f64_16x16x4f64(av[0], bv[0], acc, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(av[1], bv[1], acc1, 0, 0, 0);
        acc2 = __builtin_amdgcn_mfma_f64_16x16x4f64(av[2], bv[2], acc2, 0, 0, 0);
        acc3 = __builtin_amdgcn_mfma_f64_16x16x4f64(av[3], bv[3], acc3, 0, 0, 0);
      };
      if (RM > 24 && nrows == 128) {
        // fully unrolled, as in gram_rows_mfma: no loop-carried accumulators
#pragma unroll
        for (int k0 = 0; k0 < 128; k0 += 16) step(k0);
      } else {
        for (int k0 = 0; k0 < nrows; k0 += 16) step(k0);
      }
      acc = (acc + acc1) + (acc2 + acc3);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c1 = 16 * ta + 4 * e + g, c2 = 16 * tb + n;
        if (c1 < r && c2 < r) {
          Gs[c1 * RM + c2] = acc[e];
          Gs[c2 * RM + c1] = acc[e];
        }
      }
    }
}

// Gs = S^T S (c1, c2 < r) over nrows rows of S [nrows][RM] (nrows a multiple
// of 32) in fp64 on MFMA, the rows split over the four waves: wave w takes
// rows [w, w+1) * nrows / 4 and every upper-triangular 16x16 tile, with two
// accumulators per tile (alternate 4-row steps).  The partial sums meet in
// `slab` (2 * NT * 256 doubles, NT tiles) in a fixed order:
// (w0 + w2) + (w1 + w3).
template <int RM>
__device__ __forceinline__ void gram_rows_mfma(const float* S, int nrows, int r, double* Gs, double* slab) {
  S = lds_base(S);
  Gs = lds_base(Gs);
  slab = lds_base(slab);
  constexpr int CT = (RM + 15) / 16;
  constexpr int NT = CT * (CT + 1) / 2;
  static_assert(kThreads == 256, "four waves");
  static_assert(2 * NT * 256 * sizeof(double) <= sizeof(float) * (128 * RM + RM * RM),
                "the two slabs fit the Zs + Wf region");
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15, w = threadIdx.x >> 6;
  double4_t acc[2][NT];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) acc[u][ti] = (double4_t){0.0, 0.0, 0.0, 0.0};
  auto step = [&](int k0) __attribute__((always_inline)) {
    double v[2][CT];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        v[u][ct] = 16 * ct + n < RM ? (double)S[(k0 + 4 * u + g) * RM + min(16 * ct + n, RM - 1)] : 0.0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      int ti = 0;
#pragma unroll
      for (int ta = 0; ta < CT; ++ta)
#pragma unroll
        for (int tb = ta; tb < CT; ++tb, ++ti)
          acc[u][ti] = __builtin_amdgcn_mfma_f64_16x16x4f64(v[u][ta], v[u][tb], acc[u][ti], 0, 0, 0);
    }
  };
  if (nrows == kMaxRows) {
    // fully unrolled: every step's loads can be issued ahead of the MFMAs
    // before them, and no accumulator is loop-carried (at one wave per
    // SIMD the compiler would copy loop-carried MFMA results between the
    // register files around every step)
#pragma unroll
    for (int i = 0; i < kMaxRows / 32; ++i) step(w * (kMaxRows / 4) + 8 * i);
  } else {
    const int rpw = nrows / 4;
    for (int k0 = w * rpw; k0 < (w + 1) * rpw; k0 += 8) step(k0);
  }
#pragma unroll
  for (int ti = 0; ti < NT; ++ti) acc[0][ti] = acc[0][ti] + acc[1][ti];
  auto slab_at = [&](int sb, int ti) __attribute__((always_inline)) {
    return reinterpret_cast<double4_t*>(slab + ((sb * NT + ti) * 64 + lane) * 4);
  };
  if (w >= 2)
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) *slab_at(w - 2, ti) = acc[0][ti];
  __syncthreads();
  if (w < 2)
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) acc[0][ti] = acc[0][ti] + *slab_at(w, ti);
  __syncthreads();
  if (w == 1)
#pragma unroll
    for (int ti = 0; ti < NT; ++ti) *slab_at(0, ti) = acc[0][ti];
  __syncthreads();
  if (w == 0) {
    int ti = 0;
#pragma unroll
    for (int ta = 0; ta < CT; ++ta)
#pragma unroll
      for (int tb = ta; tb < CT; ++tb, ++ti) {
        const double4_t sum = acc[0][ti] + *slab_at(0, ti);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c1 = 16 * ta + 4 * e + g, c2 = 16 * tb + n;
          if (c1 < r && c2 < r) {
            Gs[c1 * RM + c2] = sum[e];
            Gs[c2 * RM + c1] = sum[e];
          }
        }
      }
  }
}

// Orders the LDS writes of a wave before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ double rsqrt64(double x) {
  double y = __builtin_amdgcn_rsq(x);
  y = y * fma(-0.5 * x * y, y, 1.5);
  return y * fma(-0.5 * x * y, y, 1.5);
}

// A double moved across lanes by the DPP control CTRL (both halves).
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
  const long long u = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(u & 0xffffffffLL), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(u >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// op over the 64 lanes of a wave for doubles, the result in every lane: DPP
// quad permutes, row half-mirror and row mirror (every 16-lane row), then
// permlane32 / permlane16 swaps between rows (VALU only, no LDS).
template <class Op>
__device__ __forceinline__ double wave_reduce_d(double v, Op op) {
  v = op(v, dpp_d<0xB1>(v));
  v = op(v, dpp_d<0x4E>(v));
  v = op(v, dpp_d<0x141>(v));
  v = op(v, dpp_d<0x140>(v));
  auto swap_op = [&](double x, bool wide) __attribute__((always_inline)) {
    const long long u = __double_as_longlong(x);
    const uint32_t lo = (uint32_t)(u & 0xffffffffLL), hi = (uint32_t)(u >> 32);
    auto a = wide ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                  : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    auto b = wide ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                  : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const double x0 = __longlong_as_double(((long long)b[0] << 32) | a[0]);
    const double x1 = __longlong_as_double(((long long)b[1] << 32) | a[1]);
    return op(x0, x1);
  };
  v = swap_op(v, true);
  return swap_op(v, false);
}

// Wave-uniform copy of lane `src`'s double (src a compile-time or uniform index).
__device__ __forceinline__ double lane_bcast(double v, int src) {
  const long long u = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)(u & 0xffffffffLL), src);
  const int hi = __builtin_amdgcn_readlane((int)(u >> 32), src);
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}

// Step JC of the Cholesky factorisation in cholesky_inv_wave: lane i holds
// row i of the trailing matrix; column JC is scaled by the pivot and the
// rank-1 update applied to the columns after it.  The broadcasts of L[k][JC]
// go in groups of 8, each group's readlanes issued before its FMAs (one
// SGPR pair per value, no stall between a readlane and its use).
template <int RM, int JC>
__device__ __forceinline__ void chol_col(double (&row)[RM], int lane, int r, double tol, double& il_own) {
  if (JC >= r) return;  // wave-uniform
  const double piv = lane_bcast(row[JC], JC);
  const bool dead = !(piv > tol);
  const double il = dead ? 0.0 : rsqrt64(piv);
  if (lane > JC) row[JC] *= il;                     // L[lane][JC]
  if (lane == JC) {
    row[JC] = dead ? 0.0 : piv * il;                // L[JC][JC] = sqrt(piv)
    il_own = il;
  }
  // the multiplier is zeroed on lanes <= JC, so the FMAs need no select
  const double lm = lane > JC ? -row[JC] : 0.0;
#pragma unroll
  for (int k0 = (JC + 1) & ~7; k0 < RM; k0 += 8) {
    double lk[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u > JC && k0 + u < RM) lk[u] = lane_bcast(row[JC], k0 + u);  // L[k][JC]
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (k0 + u > JC && k0 + u < RM) row[k0 + u] = fma(lm, lk[u], row[k0 + u]);
  }
}

// Step M of the forward substitution in cholesky_inv_wave, for the columns
// n = 4 j + w of L^{-1} that wave w computes (y[j] = L^{-1}[lane][n]):
// lane M finishes its entries; the lanes after it subtract L[lane][M]
// times them.  Entries with n > M are still zero, so only j <= M / 4 can
// carry anything (a zero broadcast where 4 j + w > M adds nothing).
template <int RM, int M>
__device__ __forceinline__ void inv_row(double (&y)[RM / 4], const double (&row)[RM], int lane, int w, int r,
                                        double il_own) {
  if (M >= r) return;  // wave-uniform: rows r.. of L are zero, their rows of L^{-1} too
  constexpr int JM = M / 4;
  if (lane == M) {
#pragma unroll
    for (int j = 0; j <= JM; ++j) y[j] = ((4 * j + w == M ? 1.0 : 0.0) - y[j]) * il_own;
  }
  const double lim = lane > M ? row[M] : 0.0;  // L[lane][M]; 0 leaves the finished rows unchanged
#pragma unroll
  for (int j0 = 0; j0 <= JM; j0 += 8) {
    double ym[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (j0 + u <= JM) ym[u] = lane_bcast(y[j0 + u], M);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (j0 + u <= JM) y[j0 + u] = fma(lim, ym[u], y[j0 + u]);
  }
}

// The steps as one fold over a compile-time index sequence (straight-line
// code with static register indices, not a loop left to the unroller).
template <int RM, int... J>
__device__ __forceinline__ void chol_cols(double (&row)[RM], int lane, int r, double tol, double& il_own,
                                          std::integer_sequence<int, J...>) {
  (chol_col<RM, J>(row, lane, r, tol, il_own), ...);
}
template <int RM, int... M>
__device__ __forceinline__ void inv_rows(double (&y)[RM / 4], const double (&row)[RM], int lane, int w, int r,
                                         double il_own, std::integer_sequence<int, M...>) {
  (inv_row<RM, M>(y, row, lane, w, r, il_own), ...);
}

// Cholesky G = L L^T of Gs (r x r, r <= RM) and X = R^{-1} with R = L^T.
// Wave 0 factorises: lane i keeps row i of L in registers; the steps are
// straight-line code, so register indices are static, and values move
// between lanes by readlane (no LDS, no barrier inside).  Dead columns
// (pivot <= 1e-26 of the largest diagonal entry) get L[:, j] = 0 and
// X[:, j] = 0.  L goes to LDS (transposed, over Gs) with 1 / L[i][i] in
// ilbuf; then every wave reloads it and wave w forms the columns n = 4 j + w
// of L^{-1}, lane i its row i, by forward substitution against the rows of
// the lanes before it (each element sees the same operations in the same
// order as a one-wave substitution), and writes them as column i of X
// (fp32, row-major [RM][RM], upper triangular) into Xf.
template <int RM>
__device__ __forceinline__ void cholesky_inv_wave(double* Gs, float* Xf, double* ilbuf, int r) {
  static_assert(RM % 4 == 0 && kThreads == 256, "four waves, RM / 4 columns each");
  // The lane index passes through an empty asm so that the per-step lane
  // masks below are formed in this call, not hoisted out of the caller's
  // loops as ~2*RM live 64-bit masks (which would spill).
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));
  const bool act = lane < r;
  if (threadIdx.x < 64) {
    double row[RM];
#pragma unroll
    for (int k = 0; k < RM; ++k) row[k] = (act && k < r) ? Gs[lane * RM + k] : 0.0;
    // largest diagonal entry (the diagonal read once more from LDS: a
    // lane's own entry sits at a lane-dependent register index)
    const double gm = wave_reduce_d(act ? Gs[lane * RM + lane] : 0.0,
                                    [](double a, double b) __attribute__((always_inline)) { return fmax(a, b); });
    const double tol = gm * 1e-26 + 1e-300;
    double il_own = 0.0;  // 1 / L[lane][lane] (0 when dead)
    chol_cols<RM>(row, lane, r, tol, il_own, std::make_integer_sequence<int, RM>{});
    wave_sync();  // every lane's reads of Gs are done
    if (lane < RM) {
#pragma unroll
      for (int k = 0; k < RM; ++k) Gs[k * RM + lane] = row[k];  // L^T: lane-consecutive, no bank conflicts
      ilbuf[lane] = il_own;
    }
  }
  __syncthreads();
  {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    double row[RM];
#pragma unroll
    for (int k = 0; k < RM; ++k) row[k] = lane < RM ? Gs[k * RM + min(lane, RM - 1)] : 0.0;
    const double il_own = lane < RM ? ilbuf[min(lane, RM - 1)] : 0.0;
    // y[j] = L^{-1}[lane][4 j + w]: (delta(lane, n) - sum_{m<lane} L[lane][m] L^{-1}[m][n]) / L[lane][lane]
    double y[RM / 4];
#pragma unroll
    for (int j = 0; j < RM / 4; ++j) y[j] = 0.0;
    inv_rows<RM>(y, row, lane, w, r, il_own, std::make_integer_sequence<int, RM>{});
    // X[n][lane] = L^{-1}[lane][n]
    if (lane < RM) {
#pragma unroll
      for (int j = 0; j < RM / 4; ++j) {
        const int n = 4 * j + w;
        Xf[n * RM + lane] = (act && n <= lane) ? (float)y[j] : 0.f;
      }
    }
  }
  __syncthreads();
}

// Maximum over the 64 lanes of a wave, in every lane (as wave_sum_dpp).
__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  return max_over_rows(v);
}

// Sum over the 64 lanes of a wave: DPP quad permutes, row half-mirror and
// row mirror (every 16-lane row), then permlane32 / permlane16 swaps.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  return sum_over_rows(v);
}

// Columns c < r of Ys [rows][RM] scaled to unit Euclidean norm (a column
// of zeros stays zero; columns >= r are zero).  Thread t holds rows t and
// t + kThreads in registers; the squares of each column are summed over a
// wave's lanes with DPP and permlane reductions and over the four waves in
// a fixed order.  part: >= (kThreads / 64 + 1) * RM floats of scratch.
template <int RM>
__device__ __forceinline__ void normalize_cols(float* Ys, int rows, int r, float* part) {
  static_assert(RM % 4 == 0 && kMaxRows <= 2 * kThreads, "two rows per thread, float4 columns");
  Ys = lds_base(Ys);
  part = lds_base(part);
  constexpr int NW = kThreads / 64;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const bool va = t < rows, vb = t + kThreads < rows;
  float ya[RM], yb[RM];
#pragma unroll
  for (int c = 0; c < RM; c += 4) {
    const float4 a4 = va ? *reinterpret_cast<const float4*>(Ys + t * RM + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 b4 = vb ? *reinterpret_cast<const float4*>(Ys + (t + kThreads) * RM + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    ya[c] = a4.x; ya[c + 1] = a4.y; ya[c + 2] = a4.z; ya[c + 3] = a4.w;
    yb[c] = b4.x; yb[c + 1] = b4.y; yb[c + 2] = b4.z; yb[c + 3] = b4.w;
  }
#pragma unroll
  for (int c = 0; c < RM; ++c) {
    const float sq = wave_sum_dpp(fmaf(yb[c], yb[c], ya[c] * ya[c]));
    if (lane == 0) part[w * RM + c] = sq;
  }
  __syncthreads();
  if (t < RM) {
    float nn = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) nn += part[ww * RM + t];
    part[NW * RM + t] = (t < r && nn > 0.f) ? 1.0f / sqrtf(nn) : 0.f;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < RM; c += 4) {
    const float4 s4 = *reinterpret_cast<const float4*>(part + NW * RM + c);
    if (va)
      *reinterpret_cast<float4*>(Ys + t * RM + c) = make_float4(ya[c] * s4.x, ya[c + 1] * s4.y, ya[c + 2] * s4.z, ya[c + 3] * s4.w);
    if (vb)
      *reinterpret_cast<float4*>(Ys + (t + kThreads) * RM + c) =
          make_float4(yb[c] * s4.x, yb[c + 1] * s4.y, yb[c + 2] * s4.z, yb[c + 3] * s4.w);
  }
}

// Rows of Ys <- rows of Ys X (X upper triangular, fp32 in Xf).  Thread t
// takes rows t and t + kThreads together (kept in registers), so each
// float4 of X read from LDS (a broadcast) serves both.  Output columns go
// four at a time, unrolled, so the triangle (X[m][c] = 0 for m > c) is
// skipped at compile time with no branches; a scheduling barrier after each
// group bounds the loads in flight.  No dependency chain across columns.
template <int RM>
__device__ __forceinline__ void apply_rinv(float* Ys, int rows, const float* Xf) {
  static_assert(RM % 4 == 0 && kMaxRows <= 2 * kThreads, "two rows per thread, float4 columns");
  Ys = lds_base(Ys);
  Xf = lds_base(Xf);
  const int t = threadIdx.x;
  const bool va = t < rows, vb = t + kThreads < rows;
  float ya[RM], yb[RM];
#pragma unroll
  for (int c = 0; c < RM; c += 4) {
    const float4 a4 = va ? *reinterpret_cast<const float4*>(Ys + t * RM + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 b4 = vb ? *reinterpret_cast<const float4*>(Ys + (t + kThreads) * RM + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    ya[c] = a4.x; ya[c + 1] = a4.y; ya[c + 2] = a4.z; ya[c + 3] = a4.w;
    yb[c] = b4.x; yb[c + 1] = b4.y; yb[c + 2] = b4.z; yb[c + 3] = b4.w;
  }
  auto group = [&](int c, int m) __attribute__((always_inline)) {  // row m's share of columns c..c+3
    const float4 x4 = *reinterpret_cast<const float4*>(Xf + m * RM + c);
    float4 d;
    d.x = x4.x;
    d.y = x4.y;
    d.z = x4.z;
    d.w = x4.w;
    return d;
  };
  auto fma4 = [](float4& q, float y, const float4& x) __attribute__((always_inline)) {
    q.x = fmaf(y, x.x, q.x);
    q.y = fmaf(y, x.y, q.y);
    q.z = fmaf(y, x.z, q.z);
    q.w = fmaf(y, x.w, q.w);
  };
#pragma unroll
  for (int c = 0; c < RM; c += 4) {
    float4 qa = make_float4(0.f, 0.f, 0.f, 0.f), qb = qa;
#pragma unroll
    for (int m = 0; m < c + 4; ++m) {  // X[m][c..c+3] = 0 for m >= c + 4
      const float4 x4 = group(c, m);
      fma4(qa, ya[m], x4);
      fma4(qb, yb[m], x4);
    }
    if (va) *reinterpret_cast<float4*>(Ys + t * RM + c) = qa;
    if (vb) *reinterpret_cast<float4*>(Ys + (t + kThreads) * RM + c) = qb;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Players p < q of round-robin pair m (P players, P even), advanced one
// round at a time without division: player 0 sits at circle position 0,
// the others occupy positions 1..P-1 and move one position per round
// (wrapping over the P - 1 moving slots); pair m is positions m and
// P - 1 - m.
struct PairWalk {
  int a, b, wrap;  // moving-slot indices (a < 0: fixed player 0); wrap = P - 1
  __device__ __forceinline__ void start(int P, int m) {
    wrap = P - 1;
    a = m == 0 ? -1 : m - 1;
    b = P - 2 - m;
  }
  __device__ __forceinline__ void players(int& pp, int& qq) const {
    const int x = a < 0 ? 0 : a + 1, y = b + 1;
    pp = x < y ? x : y;
    qq = x < y ? y : x;
  }
  __device__ __forceinline__ void next() {
    if (a >= 0) a = a + 1 == wrap ? 0 : a + 1;
    b = b + 1 == wrap ? 0 : b + 1;
  }
};

// Jacobi rotation (c, s) that zeroes G[p][q], branch-free: tau in fp64
// (scale-free; one Newton step on the reciprocal estimate is ample for the
// fp32 angle), the angle in fp32, then (c, s) renormalised in fp64 by one
// Newton step, so c^2 + s^2 = 1 to ~1e-14.  apq = 0 (tau inf or NaN) gives
// the identity.  An fp32 angle leaves ~1e-7 of G[p][q] behind, which the
// next sweep removes.
__device__ __forceinline__ void jacobi_rotation(double app, double aqq, double apq, double& c, double& sn) {
  const double d2 = 2.0 * apq;
  double y = __builtin_amdgcn_rcp(d2);
  y = fma(y, fma(-d2, y, 1.0), y);
  const float tau = (float)((aqq - app) * y);
  const float at = fabsf(tau);
  const float t_mid = copysignf(__builtin_amdgcn_rcpf(at + __builtin_amdgcn_sqrtf(fmaf(tau, tau, 1.0f))), tau);
  const float t_big = __builtin_amdgcn_rcpf(2.0f * tau);
  float tt = at > 1e18f ? t_big : t_mid;
  tt = apq != 0.0 ? tt : 0.0f;
  const float c32 = __builtin_amdgcn_rsqf(fmaf(tt, tt, 1.0f));
  const double cd = (double)c32, sd = (double)(tt * c32);
  const double f = fma(-0.5, fma(cd, cd, sd * sd), 1.5);
  c = cd * f;
  sn = sd * f;
}

// Cyclic parallel Jacobi on the symmetric r x r Gram in Gs (row-major,
// stride RM) by the whole workgroup.  On return Gs[i][i] holds eigenvalue i
// (the rest of Gs, and G2, are garbage) and Ws holds the eigenvectors
// transposed: Ws[i * P + c] = W[c][i] (row i is eigenvector i), P = r
// rounded up to even; Ws beyond its P x P entries is zero.
//
// Round-robin pairing over P players at fixed positions: in every round
// pair m sits at positions (m, P - 1 - m); between rounds the player at
// position x >= 1 moves to position x + 1 (P - 1 wraps to 1), so after the
// P - 1 rounds of a sweep every player is back at its start and every pair
// has met once.  The matrix is kept in position coordinates, upper triangle
// only (element (x, y) at min * P + max), double-buffered (Gs, G2): a round
// rotates the pairs in place of the positions and writes each element to
// its moved position in the other buffer.  So every thread reads and writes
// the same LDS offsets in every round, computed once; a round is one
// barrier-separated step.  A padded player's row and column are zero, so
// its rotations are the identity.  In a round every thread first issues its
// reads, then:
//   * each wave computes the rotations (c, s) of all pairs, lane l taking
//     pair l % NP (every wave computes the same values from the same
//     entries); every lane stores its pair's rotation in the wave's own slot
//     of rot (lanes of one pair store the same value) and the wave's lanes
//     read back those they need (no barrier);
//   * thread i < NB rotates the 2x2 block (pair mi, pair mk), mi <= mk, from
//     both sides (G <- J^T G J) into the other buffer (a diagonal block has
//     three distinct entries);
//   * the (pair m, row c) items of the eigenvector update, m * P + c = t,
//     t + kThreads, ..., rotate entries (players of m, c) of Ws in place
//     (at RM = 40 one round later, off the rotation chain); the players of a
//     position move by one per round, so the two LDS offsets of an item are
//     updated by one compare and select each.
// Stops at a sweep boundary when the off-diagonal mass is <= 1e-8 of the
// diagonal mass (the off-diagonal norm below 1e-4 of the diagonal's, a fifth
// of one fp16 rounding of the stored basis): the eigenvectors then mix the
// retained and the dropped directions by ~1e-4, which moves the
// reconstruction error of the truncated fit by ~1e-8 relative (second
// order), far below the fp16 and INT8 rounding of the outputs.
// scratch: >= 2 * kThreads / 64 doubles; rot: >= kThreads / 64 * RM / 2
// (c, s) pairs, 16-byte aligned.
template <int RM>
__device__ __forceinline__ void jacobi_eig(double* Gs, double* G2, double* Ws, double* scratch, double2* rot, int r) {
  static_assert(RM % 2 == 0, "even player count");
  constexpr int NP = RM / 2;
  constexpr int NB = NP * (NP + 1) / 2;  // upper-triangular 2x2 blocks
  constexpr int NW = kThreads / 64;
  constexpr int WJ = (NP * RM + kThreads - 1) / kThreads;  // eigenvector items per thread, at most
  static_assert(NB <= kThreads && NP <= 64 && 2 * NW <= 128, "one block per thread; one pair per lane");
  // Branch-free rounds for RM = 40 (one workgroup per CU, registers to
  // spare); at RM = 24 the unused lanes are masked instead, which keeps the
  // kernel within the 256 VGPRs of two workgroups per CU.
  constexpr bool BF = RM > 24;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int P = r + (r & 1), NPr = P / 2, NBr = NPr * (NPr + 1) / 2;
  double* part = scratch;  // [NW][2] partial sums
  double2* wrot = rot + w * NP;
  auto at = [P](int x, int y) __attribute__((always_inline)) { return min(x, y) * P + max(x, y); };
  auto mv = [P](int x) __attribute__((always_inline)) { return x == 0 ? 0 : (x == P - 1 ? 1 : x + 1); };
  for (int e = t; e < RM * RM; e += kThreads) {  // all of Ws: its readers take whole rows of RM entries
    const int i = e / P, k = e % P;
    Ws[e] = (e < P * P && i == k) ? 1.0 : 0.0;
    if (e < P * P && i <= k) G2[e] = (k < r) ? Gs[i * RM + k] : 0.0;
  }
  // fixed offsets: the rotation entries of pair l % NP, the block's reads
  // and its moved writes
  const int mr = lane % NPr;
  const int o_pp = at(mr, mr), o_qq = at(P - 1 - mr, P - 1 - mr), o_pq = at(mr, P - 1 - mr);
  const bool blk = t < NBr;
  const int sink = RM * RM + lane;  // BF: this lane's spare slot (same offset in Gs, G2 and Ws)
  int mi = 0, mk = 0;
  if (blk) {
    mk = (int)((sqrtf(8.0f * (float)t + 1.0f) - 1.0f) * 0.5f);  // t = mk (mk + 1) / 2 + mi
    if ((mk + 1) * (mk + 2) / 2 <= t) ++mk;
    if (mk * (mk + 1) / 2 > t) --mk;
    mi = t - mk * (mk + 1) / 2;
  }
  const int xi = mi, yi = P - 1 - mi, xk = mk, yk = P - 1 - mk;
  const int r00 = at(xi, xk), r01 = at(xi, yk), r10 = at(yi, xk), r11 = at(yi, yk);
  // BF: threads without a block (and a diagonal block's mirror) store to the sink
  const bool snk = BF && !blk;
  const int w00 = snk ? sink : at(mv(xi), mv(xk)), w01 = snk ? sink : at(mv(xi), mv(yk));
  const int w10 = snk || (BF && mi == mk) ? sink : at(mv(yi), mv(xk)), w11 = snk ? sink : at(mv(yi), mv(yk));
  // eigenvector items (pair m, row c): LDS offsets of (player at position m, c)
  // and (player at position P - 1 - m, c); player 0 never moves
  const int nitem = NPr * P;
  int im[WJ], op[WJ], oq[WJ];
  bool iv[WJ];
#pragma unroll
  for (int jj = 0; jj < WJ; ++jj) {
    const int e = t + jj * kThreads;
    iv[jj] = e < nitem;
    const int m = iv[jj] ? e / P : 0, c = iv[jj] ? e % P : 0;
    im[jj] = m;
    op[jj] = BF && !iv[jj] ? sink : m * P + c;  // BF: items beyond nitem read and write the sink
    oq[jj] = BF && !iv[jj] ? sink : (P - 1 - m) * P + c;
  }
  // PIPE (RM = 40): the eigenvector update of a round is applied one round
  // later (W never feeds the rotations), off the critical path of the next
  // round's rotations: pr/pop/poq hold the pending rotation and offsets of
  // each item, initially the identity at the first round's offsets.  At
  // RM = 24 (fewer items per thread) the update stays in its own round.
  constexpr bool PIPE = RM > 24;
  double2 pr[WJ];
  int pop[WJ], poq[WJ];
#pragma unroll
  for (int jj = 0; jj < WJ; ++jj) {
    pr[jj] = make_double2(1.0, 0.0);
    pop[jj] = op[jj];
    poq[jj] = oq[jj];
  }
  auto w_update = [&](const double2 (&rot)[WJ], const int (&o1)[WJ], const int (&o2)[WJ], const double (&vp)[WJ],
                      const double (&vq)[WJ]) __attribute__((always_inline)) {
#pragma unroll
    for (int jj = 0; jj < WJ; ++jj) {
      if (BF || iv[jj]) {
        Ws[o1[jj]] = rot[jj].x * vp[jj] - rot[jj].y * vq[jj];
        Ws[o2[jj]] = rot[jj].y * vp[jj] + rot[jj].x * vq[jj];
      }
    }
  };
  double* cur = G2;
  double* nxt = Gs;
  auto round = [&](const double* gc, double* gn) __attribute__((always_inline)) {
    // Every load is unconditional (a thread without a block reads pair 0's,
    // an item beyond the last reads offset 0), so each round has two LDS
    // round trips: the entries, then the rotations.  BF: no branches at all
    // -- what a thread must not store goes to its sink.  Otherwise the
    // unused stores are skipped by lane masks.
    const double app = gc[o_pp], aqq = gc[o_qq], apq = gc[o_pq];
    const double a00 = gc[r00], a01 = gc[r01], a10 = gc[r10], a11 = gc[r11];
    double vp[WJ], vq[WJ];  // PIPE: the pending update's entries; else this round's
#pragma unroll
    for (int jj = 0; jj < WJ; ++jj) {
      vp[jj] = Ws[PIPE ? pop[jj] : op[jj]];
      vq[jj] = Ws[PIPE ? poq[jj] : oq[jj]];
    }
    double c0, s0;
    jacobi_rotation(app, aqq, apq, c0, s0);
    wrot[mr] = make_double2(c0, s0);  // lanes >= NPr rewrite their pair's slot with the same value
    wave_sync();
    const double2 ri = wrot[mi], rk = wrot[mk];
    double2 rm[WJ];
#pragma unroll
    for (int jj = 0; jj < WJ; ++jj) rm[jj] = wrot[im[jj]];
    {
      const double ci = ri.x, si = ri.y, ck = rk.x, sk = rk.y;
      const double b00 = ci * a00 - si * a10, b01 = ci * a01 - si * a11;  // rows: J^T A
      const double b10 = si * a00 + ci * a10, b11 = si * a01 + ci * a11;
      const double n00 = ck * b00 - sk * b01, n01 = sk * b00 + ck * b01;  // columns: (J^T A) J
      const double n10 = ck * b10 - sk * b11, n11 = sk * b10 + ck * b11;
      if (BF || blk) {
        gn[w00] = n00;
        gn[w01] = n01;
        gn[w11] = n11;
        if (BF || mi != mk) gn[w10] = n10;  // a diagonal block's (y, x) is its (x, y) (BF: w10 is the sink)
      }
    }
    if constexpr (PIPE) {
      w_update(pr, pop, poq, vp, vq);  // the previous round's
#pragma unroll
      for (int jj = 0; jj < WJ; ++jj) {
        pr[jj] = rm[jj];  // this round's, applied next round
        pop[jj] = op[jj];
        poq[jj] = oq[jj];
      }
    } else {
      w_update(rm, op, oq, vp, vq);
    }
#pragma unroll
    for (int jj = 0; jj < WJ; ++jj) {
      // next round's players: p -> p - 1 (1 -> P - 1), player 0 fixed (BF:
      // sinks stay; otherwise an item beyond nitem, read but never stored,
      // keeps offsets inside the P x P entries: oq cycles through P .. (P-1) P)
      const int np = op[jj] < 2 * P ? op[jj] + (P - 2) * P : op[jj] - P;
      const int nq = oq[jj] < 2 * P ? oq[jj] + (P - 2) * P : oq[jj] - P;
      if constexpr (BF) {
        op[jj] = iv[jj] && im[jj] != 0 ? np : op[jj];
        oq[jj] = iv[jj] ? nq : oq[jj];
      } else {
        if (im[jj] != 0) op[jj] = np;
        oq[jj] = nq;
      }
    }
    __syncthreads();
  };
  // stopping test: which of this thread's entries t, t + kThreads, ... are
  // diagonal / upper (formed once, no division per sweep)
  constexpr int KE = (RM * RM + kThreads - 1) / kThreads;
  uint32_t dmask = 0, umask = 0;
#pragma unroll
  for (int ke = 0; ke < KE; ++ke) {
    const int e = t + kThreads * ke;
    if (e < P * P) {
      const int i = e / P, k = e % P;
      dmask |= (i == k ? 1u : 0u) << ke;
      umask |= (i < k ? 1u : 0u) << ke;
    }
  }
  __syncthreads();
  for (int sweep = 0; sweep < 30; ++sweep) {
    double off = 0.0, dia = 0.0;
#pragma unroll
    for (int ke = 0; ke < KE; ++ke) {
      const double v = cur[min(t + kThreads * ke, P * P - 1)];
      dia += ((dmask >> ke) & 1u) ? v * v : 0.0;
      off += ((umask >> ke) & 1u) ? 2.0 * (v * v) : 0.0;
    }
    auto add = [](double a, double b) __attribute__((always_inline)) { return a + b; };
    off = wave_reduce_d(off, add);
    dia = wave_reduce_d(dia, add);
    if (lane == 0) {
      part[2 * w] = off;
      part[2 * w + 1] = dia;
    }
    __syncthreads();
    off = 0.0;
    dia = 0.0;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {  // same order in every thread: a uniform decision
      off += part[2 * ww];
      dia += part[2 * ww + 1];
    }
    if (off <= 1e-8 * dia || dia == 0.0) break;
    double* A = cur;
    double* B = nxt;
    int step = 0;
    for (; step + 1 < P - 1; step += 2) {
      round(A, B);
      round(B, A);
    }
    if (step < P - 1) {  // odd number of rounds: the sweep ends in the other buffer
      round(A, B);
      cur = B;
      nxt = A;
    }
  }
  if constexpr (PIPE) {  // the last round's eigenvector update
    double vp[WJ], vq[WJ];
#pragma unroll
    for (int jj = 0; jj < WJ; ++jj) {
      vp[jj] = Ws[pop[jj]];
      vq[jj] = Ws[poq[jj]];
    }
    w_update(pr, pop, poq, vp, vq);
  }
  // eigenvalues to the diagonal of Gs (stride RM); cur may overlap Gs
  const double ev = t < P ? cur[t * P + t] : 0.0;
  __syncthreads();
  if (t < P) Gs[t * RM + t] = ev;
  __syncthreads();
}

template <int RM>
__device__ __forceinline__ void run_matrix(const RsvdParams& p, const Job& j, int rows, int cols, int n_iter, Lds<RM>& L,
                           const float* omega_in, long dbg_index) {
  const int t = threadIdx.x;
  const int r = j.r, k = j.k;
  const int P = r + (r & 1);  // Jacobi players: the eigenvectors are rows of Ws with stride P
  const bool mf = j.dtype == SC_DTYPE_F16 && !j.rw;  // MFMA products (fp16 input, unweighted); else fp32 VALU
  // the first M Z's first row batch, requested before the sketch is drawn
  // (the block's first reads from HBM overlap the sketch generation)
  const bool pre = mf && rows == kMaxRows && cols == 128;
  RowBatch rb0;
  if (pre) load_row_batch(j, 0, rb0);
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

  auto mul_m = [&]() __attribute__((always_inline)) {  // Ys = M Zs
    if (mf) {
      gemm_rows_mfma<RM>(j, rows, cols, L.Zs, L.Ys);
    } else {
      float y0[RM], y1[RM];
      gemm_rows<RM>(j, rows, cols, L.Zs, y0, y1);
      store_rows<RM>(L.Ys, rows, y0, y1);
    }
  };
  auto mul_mt = [&]() __attribute__((always_inline)) {  // Zs = M^T Ys
    if (mf && cols == 128) {
      gemm_cols_mfma_ct<RM>(j, rows, L.Ys, L.Zs, reinterpret_cast<h16*>(L.Gs));
    } else if (mf) {
      gemm_cols_mfma<RM>(j, rows, cols, L.Ys, L.Zs, reinterpret_cast<h16*>(L.Gs));
    } else
      gemm_cols<RM>(j, rows, cols, L.Ys, L.Zs);
  };
  auto orth_ys = [&](int passes) __attribute__((always_inline)) {  // Ys <- Q of Ys (CholeskyQR passes)
    for (int ps = 0; ps < passes; ++ps) {
      __syncthreads();
      gram_rows_mfma<RM>(L.Ys, rows, r, L.Gs, reinterpret_cast<double*>(L.Zs));  // Zs, Wf: dead here
      __syncthreads();
      cholesky_inv_wave<RM>(L.Gs, L.Wf, L.red, r);  // red: dead here
      apply_rinv<RM>(L.Ys, rows, L.Wf);
    }
  };
  if (pre)
    gemm_rows_mfma<RM>(j, rows, cols, L.Zs, L.Ys, &rb0);
  else
    mul_m();
  if (n_iter > 0) {
    // The sketch is only scaled (unit columns; the span is unchanged): that
    // bounds M^T Y like an orthonormal Y would, so the fp16 hi/lo split of
    // the next product cannot overflow.  The product of each power
    // iteration is orthonormalised (one CholeskyQR pass, two for the final
    // Q, whose second pass restores orthogonality to fp32 rounding when Y is
    // rank-deficient): the subspace of M M^T applied to an orthonormal Z is
    // conditioned well enough for fp64 Cholesky, and the fit matches the
    // float64 subspace iteration with an orthonormalisation after every
    // product to ~1e-5 of its error.
    __syncthreads();
    normalize_cols<RM>(L.Ys, rows, r, L.Zs);  // Zs (the sketch) is dead after M Z
  } else {
    orth_ys(2);
  }
  for (int it = 0; it < n_iter; ++it) {
    __syncthreads();
    mul_mt();
    __syncthreads();
    mul_m();
    orth_ys(it + 1 == n_iter ? 2 : 1);
  }
  // ---- Bp^T = M^T Q
  __syncthreads();
  mul_mt();
  __syncthreads();
  gram_mfma<RM>(L.Zs, cols, r, L.Gs);  // Bp Bp^T
  __syncthreads();
  jacobi_eig<RM>(L.Gs, L.G2, L.Ws, L.red, reinterpret_cast<double2*>(L.Wf), r);  // Wf: dead here
  // The epilogue's LDS arrays through opaque bases (one base register per
  // array plus immediate offsets; several lie past the 64 KB reach of an
  // immediate at RM = 40).
  Lds<RM> E = L;
  E.Gs = lds_base(L.Gs);
  E.Ws = lds_base(L.Ws);
  E.Ys = lds_base(L.Ys);
  E.Zs = lds_base(L.Zs);
  E.Wf = lds_base(L.Wf);
  E.red = lds_base(L.red);
  E.ord = lds_base(L.ord);
  // ---- eigenvalues in descending order: lane c takes rank = #{larger, or equal with lower index}
  if (t < r) {
    const double lc = E.Gs[t * RM + t];
    int rank = 0;
#pragma unroll
    for (int b2 = 0; b2 < RM; ++b2) {  // every load in flight at once; b2 >= r masked
      const double lb = E.Gs[b2 * RM + b2];
      rank += b2 < r && ((lb > lc) || (lb == lc && b2 < t));
    }
    E.ord[rank] = t;
  }
  __syncthreads();
  // Wf[c][i] = W[c][ord_i] * S_i  (c < r, i < k; 0 elsewhere)
  for (int e = t; e < RM * RM; e += kThreads) {
    const int c = e / RM, i = e % RM;
    float v = 0.f;
    if (c < r && i < k) {
      const int oi = E.ord[i];
      v = (float)(E.Ws[oi * P + c] * sqrt(fmax(E.Gs[oi * RM + oi], 0.0)));
    }
    E.Wf[e] = v;
  }
  __syncthreads();
  // ---- coefficients, in place over the Q rows of Ys: Ys[row][i] =
  // sum_c Q[row][c] Wf[c][i] (0 for k <= i < RM), divided by the row weight
  // when weighted.  Thread t reads and overwrites only its own rows t and
  // t + kThreads; each float4 of Wf (a wave broadcast) serves both rows
  // (Q's columns >= r and Wf's rows >= r are zero).
  const bool v0 = t < rows, v1 = t + kThreads < rows;
  {
    float cf0[RM], cf1[RM];
#pragma unroll
    for (int i = 0; i < RM; ++i) cf0[i] = cf1[i] = 0.f;
    if constexpr (RM <= 24) {
      // four columns per step: two float4 row loads and 4 x RM / 4 Wf loads
      // in flight together
      const float* ya = E.Ys + t * RM;
      const float* wf = E.Wf;
#pragma unroll 1
      for (int c4 = 0; c4 < RM; c4 += 4) {
        const float4 a4 = *reinterpret_cast<const float4*>(ya + c4);  // rows t, t + kThreads < kMaxRows: in bounds
        const float4 b4 = *reinterpret_cast<const float4*>(ya + kThreads * RM + c4);
        const float qa[4] = {v0 ? a4.x : 0.f, v0 ? a4.y : 0.f, v0 ? a4.z : 0.f, v0 ? a4.w : 0.f};
        const float qb[4] = {v1 ? b4.x : 0.f, v1 ? b4.y : 0.f, v1 ? b4.z : 0.f, v1 ? b4.w : 0.f};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float q0 = qa[u], q1 = qb[u];
#pragma unroll
          for (int i = 0; i < RM; i += 4) {  // Wf[c][i] = 0 for i >= k: those accumulators stay 0
            const float4 w = *reinterpret_cast<const float4*>(wf + (c4 + u) * RM + i);
            cf0[i] = fmaf(q0, w.x, cf0[i]);
            cf0[i + 1] = fmaf(q0, w.y, cf0[i + 1]);
            cf0[i + 2] = fmaf(q0, w.z, cf0[i + 2]);
            cf0[i + 3] = fmaf(q0, w.w, cf0[i + 3]);
            cf1[i] = fmaf(q1, w.x, cf1[i]);
            cf1[i + 1] = fmaf(q1, w.y, cf1[i + 1]);
            cf1[i + 2] = fmaf(q1, w.z, cf1[i + 2]);
            cf1[i + 3] = fmaf(q1, w.w, cf1[i + 3]);
          }
        }
      }
    } else {
      // one column per step (fewer registers in flight at RM = 40); one
      // base register per array, so a step's Wf row loads are issued
      // together with immediate offsets
      const float* ya = E.Ys + t * RM;
      const float* wf = E.Wf;
#pragma unroll 1
      for (int c = 0; c < r; ++c) {
        const float a = ya[c], b = ya[kThreads * RM + c];  // rows t, t + kThreads < kMaxRows: in bounds
        const float q0 = v0 ? a : 0.f, q1 = v1 ? b : 0.f;
        const float* wr = wf + c * RM;
#pragma unroll
        for (int i = 0; i < RM; i += 4) {  // Wf[c][i] = 0 for i >= k: those accumulators stay 0
          const float4 w = *reinterpret_cast<const float4*>(wr + i);
          cf0[i] = fmaf(q0, w.x, cf0[i]);
          cf0[i + 1] = fmaf(q0, w.y, cf0[i + 1]);
          cf0[i + 2] = fmaf(q0, w.z, cf0[i + 2]);
          cf0[i + 3] = fmaf(q0, w.w, cf0[i + 3]);
          cf1[i] = fmaf(q1, w.x, cf1[i]);
          cf1[i + 1] = fmaf(q1, w.y, cf1[i + 1]);
          cf1[i + 2] = fmaf(q1, w.z, cf1[i + 2]);
          cf1[i + 3] = fmaf(q1, w.w, cf1[i + 3]);
        }
      }
    }
    if (j.rw) {  // undo the row weighting: coeffs / W (spectral_cache.py:389-393)
      const float w0 = v0 ? row_weight(j, t) : 1.f, w1 = v1 ? row_weight(j, t + kThreads) : 1.f;
#pragma unroll
      for (int i = 0; i < RM; ++i)
        if (i < k) {
          cf0[i] = cf0[i] / w0;
          cf1[i] = cf1[i] / w1;
        }
    }
    // Wf[c][i] = 0 for i >= k, so cf[i] = 0 there: whole rows are stored
#pragma unroll
    for (int i = 0; i < RM; i += 4) {
      if (v0) *reinterpret_cast<float4*>(E.Ys + t * RM + i) = make_float4(cf0[i], cf0[i + 1], cf0[i + 2], cf0[i + 3]);
      if (v1)
        *reinterpret_cast<float4*>(E.Ys + (t + kThreads) * RM + i) =
            make_float4(cf1[i], cf1[i + 1], cf1[i + 2], cf1[i + 3]);
    }
  }
  if (p.coeffs_out && dbg_index >= 0) {
    for (int i = 0; i < k; ++i) {
      if (v0) p.coeffs_out[(dbg_index * rows + t) * k + i] = E.Ys[t * RM + i];
      if (v1) p.coeffs_out[(dbg_index * rows + t + kThreads) * k + i] = E.Ys[(t + kThreads) * RM + i];
    }
  }
  // Vh (unnormalised), in place over Bp^T in Zs, as [k][cols]:
  // Vh_i[d] = sum_c W[c][ord_i] Bp^T[d][c].  Thread t owns column d = t % cols:
  // it loads its Bp^T row into registers before the barrier, then writes
  // ranks t / cols, t / cols + kThreads / cols, ...; W reads are wave
  // broadcasts.  (k cols <= 128 RM: Vh fits in Zs.)
  {
    const int d = t % cols, istep = kThreads / cols;
    float z[RM];
#pragma unroll
    for (int c = 0; c < RM; c += 4) {
      const float4 z4 = *reinterpret_cast<const float4*>(E.Zs + d * RM + c);
      z[c] = z4.x;
      z[c + 1] = z4.y;
      z[c + 2] = z4.z;
      z[c + 3] = z4.w;
    }
    __syncthreads();  // every Bp^T row is in registers
#pragma unroll 2
    for (int i = t / cols; i < k; i += istep) {
      // whole rows of RM entries, no branches: z[c] = 0 for c >= r (the
      // columns of Q beyond r are zero) and Ws is zero beyond P x P
      const double* wr = E.Ws + E.ord[i] * P;
      double a0 = 0.0, a1 = 0.0;
#pragma unroll
      for (int c = 0; c < RM; c += 2) {
        const double2 w2 = *reinterpret_cast<const double2*>(wr + c);
        a0 = fma(w2.x, (double)z[c], a0);
        a1 = fma(w2.y, (double)z[c + 1], a1);
      }
      E.Zs[i * cols + d] = (float)(a0 + a1);
    }
  }
  __syncthreads();
  for (int i = t >> 6; i < k; i += kThreads / 64) {  // row norms -> 1/norm (0 for vanished rows), one wave per row
    double nn = 0.0;
    for (int d = t & 63; d < cols; d += 64) {
      const double v = E.Zs[i * cols + d];
      nn += v * v;
    }
    nn = wave_reduce_d(nn, [](double a, double b) __attribute__((always_inline)) { return a + b; });
    if ((t & 63) == 0) {
      E.red[i] = nn > 0.0 ? 1.0 / sqrt(nn) : 0.0;
      if (p.svals_out && dbg_index >= 0) {
        const int oi = E.ord[i];
        p.svals_out[dbg_index * k + i] = (float)sqrt(fmax(E.Gs[oi * RM + oi], 0.0));
      }
    }
  }
  __syncthreads();
  // basis
  auto basis_value = [&](int i, int d) __attribute__((always_inline)) {
    return i < k ? (float)(E.Zs[i * cols + d] * E.red[i]) : 0.f;
  };
  const bool dbg_vh = p.vh_out && dbg_index >= 0;
  if (!dbg_vh && j.kp % 8 == 0 && cols % 8 == 0 && (reinterpret_cast<uintptr_t>(j.basis) & 15) == 0) {
    // eight consecutive values of the output layout per 16-byte store
    const int per = (j.basis_dmajor ? j.kp : cols) / 8;
    const int n_items = (j.basis_dmajor ? cols : j.kp) * per;
    for (int e = t; e < n_items; e += kThreads) {
      const int a = e / per, b0 = (e % per) * 8;
      half8_t h;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        h[u] = (h16)(j.basis_dmajor ? basis_value(b0 + u, a) : basis_value(a, b0 + u));  // (rank, column)
      *reinterpret_cast<half8_t*>(j.basis + (long)a * (j.basis_dmajor ? j.kp : cols) + b0) = h;
    }
  } else {
    for (int e = t; e < j.kp * cols; e += kThreads) {
      const int i = e / cols, d = e % cols;
      const float v = basis_value(i, d);
      if (j.basis_dmajor)
        j.basis[(long)d * j.kp + i] = (h16)v;
      else
        j.basis[(long)i * cols + d] = (h16)v;
      if (dbg_vh && i < k) p.vh_out[(dbg_index * k + i) * cols + d] = v;
    }
  }
  // ---- quantise (spectral_cache.py:481-516 formula); each thread re-reads
  // its own coefficient rows from Ys
  float am0 = 0.f, am1 = 0.f, mn = INFINITY, mx = -INFINITY;
  auto row_stats = [&](int row, float& am) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < RM; i += 4) {  // columns >= k hold 0: masked by selects, no branches
      const float4 c4 = *reinterpret_cast<const float4*>(E.Ys + row * RM + i);
      const float cv[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool in = i + u < k;
        am = fmaxf(am, fabsf(cv[u]));
        mn = fminf(mn, in ? cv[u] : INFINITY);
        mx = fmaxf(mx, in ? cv[u] : -INFINITY);
      }
    }
  };
  if (v0) row_stats(t, am0);
  if (v1) row_stats(t + kThreads, am1);
  // block reductions: absmax, min, max
  float* fred = (float*)E.red;
  __syncthreads();
  {
    const float wa = wave_max_dpp(fmaxf(am0, am1)), wmn = -wave_max_dpp(-mn), wmx = wave_max_dpp(mx);
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
    const float ws = wave_max_dpp(fmaxf(v0 ? s0 : 0.f, v1 ? s1 : 0.f));
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
  // row-major codes with kp a multiple of 4 and an aligned base: four
  // codes of a row per dword store
  const bool pack = !j.coeff_major && j.kp % 4 == 0 && (reinterpret_cast<uintptr_t>(j.codes) & 3) == 0;
  auto pack4 = [](const int8_t (&q)[4]) __attribute__((always_inline)) {
    return (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
           ((uint32_t)(uint8_t)q[3] << 24);
  };
#pragma unroll
  for (int i = 0; i < RM; i += 4) {
    if (i < j.kp) {
      // rows t and t + kThreads < kMaxRows: in bounds (rows past `rows`
      // are never stored); columns >= k hold 0, whose code is 0
      const float4 a4 = *reinterpret_cast<const float4*>(E.Ys + t * RM + i);
      const float4 b4 = *reinterpret_cast<const float4*>(E.Ys + (t + kThreads) * RM + i);
      const float ca[4] = {a4.x, a4.y, a4.z, a4.w}, cb[4] = {b4.x, b4.y, b4.z, b4.w};
      int8_t qa[4], qb[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        qa[u] = (int8_t)(int)rintf(ca[u] / s0);  // IEEE division, ties to even
        qb[u] = (int8_t)(int)rintf(cb[u] / s1);
      }
      if (pack) {
        if (v0) *reinterpret_cast<uint32_t*>(j.codes + (long)t * j.kp + i) = pack4(qa);
        if (v1) *reinterpret_cast<uint32_t*>(j.codes + (long)(t + kThreads) * j.kp + i) = pack4(qb);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (i + u < j.kp) put(i + u, qa[u], qb[u]);
      }
    }
  }
  if (pack) {
    for (int i = RM; i < j.kp; i += 4) {
      if (v0) *reinterpret_cast<uint32_t*>(j.codes + (long)t * j.kp + i) = 0u;
      if (v1) *reinterpret_cast<uint32_t*>(j.codes + (long)(t + kThreads) * j.kp + i) = 0u;
    }
  } else {
    for (int i = RM; i < j.kp; ++i) put(i, 0, 0);
  }
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
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(RM <= 24 ? 2 : 1))) void rsvd_generic_kernel(RsvdParams p) {
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
  j.rw = nullptr;
  j.rw_mean = 1.f;
  if (p.row_weights) {  // mean of the row importances (spectral_cache.py:357), one block reduction
    j.rw = p.row_weights + io * p.rw_so + ii * p.rw_si;
    const int t = threadIdx.x;
    float s = 0.f;
    for (int e = t; e < p.rows; e += kThreads) s += j.rw[e];
    s = wave_sum(s);
    float* fr = reinterpret_cast<float*>(L.red);
    if ((t & 63) == 0) fr[t >> 6] = s;
    __syncthreads();
    j.rw_mean = ((fr[0] + fr[1]) + (fr[2] + fr[3])) / (float)p.rows;
    __syncthreads();
  }
  run_matrix<RM>(p, j, p.rows, p.cols, p.n_iter, L, p.omega ? p.omega + i * (long)p.cols * p.r : nullptr, i);
}

// Tier mode: unit = (b, i, h, kind); compresses block i of sequence b's
// tail (if full) into cold slot NCOLD + i.
__device__ __forceinline__ int tier_new_blocks(const RsvdParams& p, const int32_t* cnt) {
  const int full = cnt[SC_CNT_TAIL_LEN] / p.tier.block_size;
  return max(0, min(min(full, p.max_new), p.NB - cnt[SC_CNT_NCOLD]));
}

template <int RM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(RM <= 24 ? 2 : 1))) void rsvd_tier_kernel(RsvdParams p) {
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
  j.rw = nullptr;
  j.rw_mean = 1.f;
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
  p.row_weights = a->row_weights;
  p.rw_so = a->row_weights_stride_outer;
  p.rw_si = a->row_weights_stride_inner;
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
