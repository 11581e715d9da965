// Decode attention over the three-tier spectral cache (gfx950).
//
// Replaces the per-block PyTorch loops of
//   spectral_attention_decode   kernels/spectral_attention.py:684-857 (absolute RoPE)
//   spectral_attention_forward  spectral_attention.py:117-349          (distance RoPE)
// with one split-K kernel plus a log-sum-exp combine.
//
// Work unit = (sequence b, KV head h, chunk).  A chunk is one cold block
// (block_size tokens) or 64 tail tokens.  A unit runs on one 256-thread
// workgroup; wave w owns a quarter of the chunk and walks it in tiles of 16
// tokens.  Per cold tile and KV head:
//   1. codes (INT8, token-major) -> fp16 in registers (exact), and
//      X^T = B_K^T . code^T on MFMA 16x16x32 (the basis of the block is
//      held in VGPRs for the whole block; its rows are permuted so that a
//      lane ends up with a token's d and d+D/2 entries -- a RoPE pair).
//   2. RoPE of the reconstructed key, in packed fp16: R_phi(x), with
//      phi = p (absolute) or max(q-p,0) (distance), cos/sin rows of the
//      caller's table.  Row scale s_t is applied after the dot (linear).
//   3. scores of the whole GQA group: S = Y . Q^T on MFMA (Q in VGPRs).
//   4. online softmax in the log2 domain, row-group butterflies.
//   5. P . C_V accumulated on MFMA 16x16x16 with the per-token V scale
//      folded into P (prescaled by the block's power-of-two vnorm), codes
//      of V stored coefficient-major so each lane reads 4 contiguous bytes.
// At the end of the block the four waves merge in LDS and the merged
// (P.C_V) of every query head is projected once through B_V.
// Tail chunks skip step 1 (fp16 keys) and use P . V directly.
#include <math.h>

#include "sc_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 16;
constexpr int kTailUnit = kWaves * kTile;  // tail tokens per unit
constexpr int kMaxRep = 16;                // query heads per KV head (MFMA N)

struct DecodeParams {
  int B, Hq, Hkv, nrep, TB, NB, TCAP, per_row, rope_mode, rope_len, halves_equal;
  int grid_blocks, tail_units, units_per_bh, total_units;
  float scale, scale_log2;
  const h16* q;
  long q_sb, q_sh;
  const int8_t* codes_k;
  const int8_t* codes_v;
  const float* scales_k;
  const float* scales_v;
  const float* vnorm;
  const h16* basis_k;
  const h16* basis_v;
  const int32_t* block_start;
  const h16* tail_k;
  const h16* tail_v;
  const int32_t* tail_pos;
  const int32_t* counters;
  const h16* cos;
  const h16* sin;
  long rope_stride;
  const int32_t* qpos;
  int qpos_scalar;
  const uint8_t* mask;
  long mask_sb, mask_sh;
  float* logits;
  long lg_sb, lg_sh;
  float* ws;
  h16* out;
  long out_sb, out_sh;
};

// Rotation variants (pairs (x1, x2) = (x[d], x[d + D/2])):
//   cold, absolute : (c1 x1 - s2 x2, s1 x1 + c2 x2)  from Q . R_{-p} (_apply_inverse_rope)
//   tail, absolute : (c1 x1 - s1 x2, s2 x1 + c2 x2)  _apply_rope on the key
//   distance       : (c1 x1 - s1 x2, s1 x1 + c1 x2)  apply_rope (first half only)
enum RotKind { kRotColdAbs = 0, kRotTailAbs = 1, kRotDist = 2 };

template <int D>
struct Geo {
  static constexpr int HALF = D / 2;
  static constexpr int QG = HALF / 4;     // pairs per lane
  static constexpr int NP = QG / 2;       // half2 pairs per lane
  static constexpr int MT = D / 16;       // 16-row tiles over d
  static constexpr int MTH = MT / 2;
  static constexpr int DS = D / 32;       // K-steps of the score MFMA
  static constexpr int PREC = D + 2;      // partial record: m, l, o[D]
};

// Loads QG consecutive fp16 (QG = 8 or 16) as half2 pairs.
template <int QG>
__device__ __forceinline__ void load_pairs(const h16* src, half2_t (&dst)[QG / 2]) {
#pragma unroll
  for (int v = 0; v < QG / 8; ++v) {
    half8_t t = *reinterpret_cast<const half8_t*>(src + 8 * v);
#pragma unroll
    for (int e = 0; e < 4; ++e) dst[4 * v + e] = (half2_t){t[2 * e], t[2 * e + 1]};
  }
}

// Rotates the lane's QG pairs in packed fp16 and packs the result as the
// A operand (per K-step of 8) of the score MFMA.
template <int D>
__device__ __forceinline__ void rotate_pairs(const half2_t (&x1)[Geo<D>::NP], const half2_t (&x2)[Geo<D>::NP],
                                             const h16* crow, const h16* srow, int g, int kind,
                                             bool halves_equal, half8_t (&ya)[Geo<D>::DS]) {
  using G = Geo<D>;
  half2_t c1[G::NP], s1[G::NP], c2[G::NP], s2[G::NP];
  load_pairs<G::QG>(crow + g * G::QG, c1);
  load_pairs<G::QG>(srow + g * G::QG, s1);
  if (!halves_equal && kind != kRotDist) {
    load_pairs<G::QG>(crow + G::HALF + g * G::QG, c2);
    load_pairs<G::QG>(srow + G::HALF + g * G::QG, s2);
  } else {
#pragma unroll
    for (int e = 0; e < G::NP; ++e) {
      c2[e] = c1[e];
      s2[e] = s1[e];
    }
  }
  half2_t y1[G::NP], y2[G::NP];
#pragma unroll
  for (int e = 0; e < G::NP; ++e) {
    const half2_t sa = (kind == kRotColdAbs) ? s2[e] : s1[e];
    const half2_t sb = (kind == kRotTailAbs) ? s2[e] : s1[e];
    const half2_t cb = (kind == kRotDist) ? c1[e] : c2[e];
    y1[e] = c1[e] * x1[e] - sa * x2[e];
    y2[e] = sb * x1[e] + cb * x2[e];
  }
#pragma unroll
  for (int s = 0; s < G::DS; ++s) {
    const half2_t* src = (s < G::DS / 2) ? &y1[4 * s] : &y2[4 * (s - G::DS / 2)];
    ya[s] = (half8_t){src[0].x, src[0].y, src[1].x, src[1].y, src[2].x, src[2].y, src[3].x, src[3].y};
  }
}

template <int D>
__device__ __forceinline__ void pack_unrotated(const half2_t (&x1)[Geo<D>::NP], const half2_t (&x2)[Geo<D>::NP],
                                               half8_t (&ya)[Geo<D>::DS]) {
  using G = Geo<D>;
#pragma unroll
  for (int s = 0; s < G::DS; ++s) {
    const half2_t* src = (s < G::DS / 2) ? &x1[4 * s] : &x2[4 * (s - G::DS / 2)];
    ya[s] = (half8_t){src[0].x, src[0].y, src[1].x, src[1].y, src[2].x, src[2].y, src[3].x, src[3].y};
  }
}

// Query operand of the score MFMA: lane (g, n) holds head n, d-slots of
// K-step s = the lane group's RoPE pairs, matching the Y layout.
template <int D>
__device__ __forceinline__ void load_q(const DecodeParams& p, int b, int h, int g, int n, bool hv,
                                       half8_t (&qb)[Geo<D>::DS]) {
  using G = Geo<D>;
  const h16* qrow = p.q + b * p.q_sb + (long)(h * p.nrep + (hv ? n : 0)) * p.q_sh;
#pragma unroll
  for (int s = 0; s < G::DS; ++s) {
    const int d0 = (s < G::DS / 2) ? g * G::QG + 8 * s : G::HALF + g * G::QG + 8 * (s - G::DS / 2);
    qb[s] = hv ? *reinterpret_cast<const half8_t*>(qrow + d0) : (half8_t)(h16)0;
  }
}

__device__ __forceinline__ float* record_ptr(const DecodeParams& p, int b, int h, int unit, int hh, int prec) {
  return p.ws + ((((long)(b * p.Hkv + h) * p.units_per_bh + unit) * p.nrep + hh) * prec);
}

__device__ __forceinline__ void write_empty(const DecodeParams& p, int b, int h, int unit, int prec) {
  if ((int)threadIdx.x < p.nrep) {
    float* r = record_ptr(p, b, h, unit, threadIdx.x, prec);
    r[0] = -INFINITY;
    r[1] = 0.f;
  }
}

__device__ __forceinline__ int clamp_angle(int phi, int len) { return min(max(phi, 0), len - 1); }

// ------------------------------------------------------------------ cold
template <int D, int KK, int KV>
__device__ void cold_unit(const DecodeParams& p, int b, int h, int j, float* lds) {
  using G = Geo<D>;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
  const int ncold = p.counters[b * SC_NCOUNTERS + SC_CNT_NCOLD];
  if (j >= ncold) {
    write_empty(p, b, h, j, G::PREC);
    return;
  }
  const int nrep = p.nrep;
  const bool hv = n < nrep;
  const long bhj = (long)(b * p.Hkv + h) * p.NB + j;
  const int start = p.block_start[b * p.NB + j];
  const int qp = p.qpos ? p.qpos[b] : p.qpos_scalar;

  half8_t qb[G::DS];
  load_q<D>(p, b, h, g, n, hv, qb);

  // Basis of K as the A operand: row n of tile mt is d = perm(mt, n).
  constexpr int KC = KK >= 32 ? KK / 32 : 1;
  half8_t a8[G::MT][KC];
  half4_t a4[G::MT];
  const h16* bk = p.basis_k + bhj * (long)D * KK;
#pragma unroll
  for (int mt = 0; mt < G::MT; ++mt) {
    const int hh = mt / G::MTH, mtl = mt % G::MTH;
    const int d = hh * G::HALF + (n >> 2) * G::QG + 4 * mtl + (n & 3);
    if constexpr (KK == 16) {
      a4[mt] = *reinterpret_cast<const half4_t*>(bk + d * KK + 4 * g);
    } else {
#pragma unroll
      for (int c = 0; c < KC; ++c) a8[mt][c] = *reinterpret_cast<const half8_t*>(bk + d * KK + c * 32 + 8 * g);
    }
  }

  const int8_t* ck = p.codes_k + bhj * (long)p.TB * KK;
  const int8_t* cv = p.codes_v + bhj * (long)KV * p.TB;
  const float* skp = p.scales_k + (p.per_row ? bhj * p.TB : bhj);
  const float* svp = p.scales_v + (p.per_row ? bhj * p.TB : bhj);
  const float vn = p.vnorm[bhj];
  const int kind = p.rope_mode == SC_ROPE_DISTANCE ? kRotDist : kRotColdAbs;
  const uint8_t* mrow = (p.mask && hv) ? p.mask + b * p.mask_sb + (long)(h * nrep + n) * p.mask_sh + (long)j * p.TB : nullptr;
  float* lrow = (p.logits && hv) ? p.logits + b * p.lg_sb + (long)(h * nrep + n) * p.lg_sh + (long)j * p.TB : nullptr;

  float m_run = -INFINITY, l_run = 0.f;
  float4_t pacc[KV / 16];
#pragma unroll
  for (int nt = 0; nt < KV / 16; ++nt) pacc[nt] = (float4_t)0.f;

  const int per_wave = p.TB / kWaves;
  const int tok0 = w * per_wave;
  for (int tb = tok0; tb < tok0 + per_wave; tb += kTile) {
    // 1. reconstruct X^T[d][token] for the 16 tokens of the tile.
    float4_t x[G::MT];
    if constexpr (KK == 16) {
      const half4_t bc = i8x4_to_h4(*reinterpret_cast<const uint32_t*>(ck + (tb + n) * KK + 4 * g));
#pragma unroll
      for (int mt = 0; mt < G::MT; ++mt) x[mt] = mfma_16x16x16(a4[mt], bc, (float4_t)0.f);
    } else {
      half8_t bc[KC];
#pragma unroll
      for (int c = 0; c < KC; ++c)
        bc[c] = i8x8_to_h8(*reinterpret_cast<const uint2*>(ck + (tb + n) * KK + c * 32 + 8 * g));
#pragma unroll
      for (int mt = 0; mt < G::MT; ++mt) {
        float4_t acc = (float4_t)0.f;
#pragma unroll
        for (int c = 0; c < KC; ++c) acc = mfma_16x16x32(a8[mt][c], bc[c], acc);
        x[mt] = acc;
      }
    }
    half2_t x1[G::NP], x2[G::NP];
#pragma unroll
    for (int e = 0; e < G::NP; ++e) {
      const int mt = (2 * e) >> 2, jj = (2 * e) & 3;
      x1[e] = pack_h2(x[mt][jj], x[mt][jj + 1]);
      x2[e] = pack_h2(x[G::MTH + mt][jj], x[G::MTH + mt][jj + 1]);
    }
    // 2. RoPE of token tb + n.
    half8_t ya[G::DS];
    if (p.rope_mode == SC_ROPE_NONE) {
      pack_unrotated<D>(x1, x2, ya);
    } else {
      const int pos = start + tb + n;
      const int phi = clamp_angle(p.rope_mode == SC_ROPE_DISTANCE ? max(qp - pos, 0) : pos, p.rope_len);
      rotate_pairs<D>(x1, x2, p.cos + phi * p.rope_stride, p.sin + phi * p.rope_stride, g, kind,
                      p.halves_equal != 0, ya);
    }
    // 3. scores of the GQA group: lane holds head n, tokens tb + 4g + jj.
    float4_t sacc = (float4_t)0.f;
#pragma unroll
    for (int s = 0; s < G::DS; ++s) sacc = mfma_16x16x32(ya[s], qb[s], sacc);
    const float4_t sk4 = p.per_row ? *reinterpret_cast<const float4_t*>(skp + tb + 4 * g) : (float4_t)skp[0];
    float sc[4];
    uint32_t keep = 0xffffffffu;
    if (mrow) keep = *reinterpret_cast<const uint32_t*>(mrow + tb + 4 * g);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float raw = sacc[jj] * sk4[jj];
      if (lrow) lrow[tb + 4 * g + jj] = raw * p.scale;
      const bool k = hv && ((keep >> (8 * jj)) & 0xffu);
      sc[jj] = k ? raw * p.scale_log2 : -INFINITY;
    }
    // 4. online softmax (log2 domain).
    const float tmax = max_over_rows(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
    const float m_new = fmaxf(m_run, tmax);
    const bool live = m_new != -INFINITY;
    const float alpha = live ? exp2f(m_run - m_new) : 1.f;
    float pv[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) pv[jj] = live ? exp2f(sc[jj] - m_new) : 0.f;
    l_run = l_run * alpha + sum_over_rows(pv[0] + pv[1] + pv[2] + pv[3]);
    m_run = m_new;
    // 5. Pacc^T[i][head] += C_V^T[i][tok] . (P s_V vnorm)[tok][head]
    const float4_t sv4 = p.per_row ? *reinterpret_cast<const float4_t*>(svp + tb + 4 * g) : (float4_t)svp[0];
    const half4_t pb = {(h16)(pv[0] * sv4[0] * vn), (h16)(pv[1] * sv4[1] * vn), (h16)(pv[2] * sv4[2] * vn),
                        (h16)(pv[3] * sv4[3] * vn)};
#pragma unroll
    for (int nt = 0; nt < KV / 16; ++nt) {
      const half4_t ca = i8x4_to_h4(*reinterpret_cast<const uint32_t*>(cv + (long)(nt * 16 + n) * p.TB + tb + 4 * g));
      pacc[nt] = mfma_16x16x16(ca, pb, pacc[nt] * alpha);
    }
  }

  // ---- merge the four waves, project through B_V once.
  float* s_m = lds;                         // [kWaves][nrep]
  float* s_l = s_m + kWaves * nrep;         // [kWaves][nrep]
  float* s_acc = s_l + kWaves * nrep;       // [kWaves][nrep][KV]
  float* s_mrg = s_acc + kWaves * nrep * KV;  // [nrep][KV]
  float* s_ml = s_mrg + nrep * KV;          // [nrep][2]
  if (hv) {
    if (g == 0) {
      s_m[w * nrep + n] = m_run;
      s_l[w * nrep + n] = l_run;
    }
#pragma unroll
    for (int nt = 0; nt < KV / 16; ++nt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) s_acc[(w * nrep + n) * KV + nt * 16 + 4 * g + jj] = pacc[nt][jj];
  }
  __syncthreads();
  const float inv_vn = 1.0f / vn;
  for (int idx = threadIdx.x; idx < nrep * KV; idx += kThreads) {
    const int hh = idx / KV, i = idx % KV;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, s_m[ww * nrep + hh]);
    float acc = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const float mw = s_m[ww * nrep + hh];
        const float a = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
        acc += a * s_acc[(ww * nrep + hh) * KV + i];
        L += a * s_l[ww * nrep + hh];
      }
    }
    s_mrg[idx] = acc * inv_vn;
    if (i == 0) {
      s_ml[2 * hh] = M;
      s_ml[2 * hh + 1] = L;
    }
  }
  __syncthreads();
  const h16* bv = p.basis_v + bhj * (long)KV * D;
  for (int idx = threadIdx.x; idx < nrep * D; idx += kThreads) {
    const int hh = idx / D, d = idx % D;
    float o = 0.f;
#pragma unroll 8
    for (int i = 0; i < KV; ++i) o += s_mrg[hh * KV + i] * (float)bv[i * D + d];
    record_ptr(p, b, h, j, hh, G::PREC)[2 + d] = o;
  }
  if ((int)threadIdx.x < nrep) {
    float* r = record_ptr(p, b, h, j, threadIdx.x, G::PREC);
    r[0] = s_ml[2 * threadIdx.x];
    r[1] = s_ml[2 * threadIdx.x + 1];
  }
}

// ------------------------------------------------------------------ tail
template <int D>
__device__ void tail_unit(const DecodeParams& p, int b, int h, int c, float* lds) {
  using G = Geo<D>;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, g = lane >> 4, n = lane & 15;
  const int unit = p.grid_blocks + c;
  const int* cnt = p.counters + b * SC_NCOUNTERS;
  const int tl = cnt[SC_CNT_TAIL_LEN], th = cnt[SC_CNT_TAIL_HEAD], ncold = cnt[SC_CNT_NCOLD];
  if (c * kTailUnit >= tl) {
    write_empty(p, b, h, unit, G::PREC);
    return;
  }
  const int nrep = p.nrep;
  const bool hv = n < nrep;
  const long bh = (long)(b * p.Hkv + h);
  const int tile0 = c * kTailUnit + w * kTile;

  half8_t qb[G::DS];
  load_q<D>(p, b, h, g, n, hv, qb);

  // Key row of token tile0 + n.
  const int t = tile0 + n;
  const bool tv = t < tl;
  const int slot = (th + (tv ? t : 0)) % p.TCAP;
  half2_t x1[G::NP], x2[G::NP];
  if (tv) {
    const h16* krow = p.tail_k + (bh * p.TCAP + slot) * D;
    load_pairs<G::QG>(krow + g * G::QG, x1);
    load_pairs<G::QG>(krow + G::HALF + g * G::QG, x2);
  } else {
#pragma unroll
    for (int e = 0; e < G::NP; ++e) x1[e] = x2[e] = (half2_t)(h16)0;
  }
  half8_t ya[G::DS];
  if (p.rope_mode == SC_ROPE_NONE) {
    pack_unrotated<D>(x1, x2, ya);
  } else {
    const int pos = tv ? p.tail_pos[(long)b * p.TCAP + slot] : 0;
    const int phi = clamp_angle(pos, p.rope_len);
    rotate_pairs<D>(x1, x2, p.cos + phi * p.rope_stride, p.sin + phi * p.rope_stride, g,
                    p.rope_mode == SC_ROPE_DISTANCE ? kRotDist : kRotTailAbs, p.halves_equal != 0, ya);
  }
  float4_t sacc = (float4_t)0.f;
#pragma unroll
  for (int s = 0; s < G::DS; ++s) sacc = mfma_16x16x32(ya[s], qb[s], sacc);

  const long cache_off = (long)ncold * p.TB;  // tail follows the cold blocks
  const uint8_t* mrow = (p.mask && hv) ? p.mask + b * p.mask_sb + (long)(h * nrep + n) * p.mask_sh + cache_off : nullptr;
  float* lrow = (p.logits && hv) ? p.logits + b * p.lg_sb + (long)(h * nrep + n) * p.lg_sh + cache_off : nullptr;
  float sc[4];
  int vslot[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) {
    const int tt = tile0 + 4 * g + jj;
    const bool valid = tt < tl;
    vslot[jj] = valid ? (th + tt) % p.TCAP : -1;
    const float raw = sacc[jj];
    if (lrow && valid) lrow[tt] = raw * p.scale;
    bool k = hv && valid;
    if (k && mrow) k = mrow[tt] != 0;
    sc[jj] = k ? raw * p.scale_log2 : -INFINITY;
  }
  const float m_w = max_over_rows(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])));
  const bool live = m_w != -INFINITY;
  float pv[4];
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) pv[jj] = live ? exp2f(sc[jj] - m_w) : 0.f;
  const float l_w = sum_over_rows(pv[0] + pv[1] + pv[2] + pv[3]);
  const half4_t pb = {(h16)pv[0], (h16)pv[1], (h16)pv[2], (h16)pv[3]};

  // O^T[d][head] = V^T[d][tok] . P[tok][head]
  float4_t oacc[G::MT];
  const h16* vbase = p.tail_v + bh * p.TCAP * D;
#pragma unroll
  for (int mt = 0; mt < G::MT; ++mt) {
    h16 va[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) va[jj] = vslot[jj] >= 0 ? vbase[(long)vslot[jj] * D + mt * 16 + n] : (h16)0;
    oacc[mt] = mfma_16x16x16((half4_t){va[0], va[1], va[2], va[3]}, pb, (float4_t)0.f);
  }

  float* s_m = lds;                    // [kWaves][nrep]
  float* s_l = s_m + kWaves * nrep;    // [kWaves][nrep]
  float* s_acc = s_l + kWaves * nrep;  // [kWaves][nrep][D]
  if (hv) {
    if (g == 0) {
      s_m[w * nrep + n] = m_w;
      s_l[w * nrep + n] = l_w;
    }
#pragma unroll
    for (int mt = 0; mt < G::MT; ++mt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) s_acc[(w * nrep + n) * D + mt * 16 + 4 * g + jj] = oacc[mt][jj];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < nrep * D; idx += kThreads) {
    const int hh = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, s_m[ww * nrep + hh]);
    float acc = 0.f, L = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const float mw = s_m[ww * nrep + hh];
        const float a = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
        acc += a * s_acc[(ww * nrep + hh) * D + d];
        L += a * s_l[ww * nrep + hh];
      }
    }
    float* r = record_ptr(p, b, h, unit, hh, G::PREC);
    r[2 + d] = acc;
    if (d == 0) {
      r[0] = M;
      r[1] = L;
    }
  }
}

template <int D, int KK, int KV>
__global__ __launch_bounds__(kThreads) void decode_partial_kernel(DecodeParams p) {
  extern __shared__ float lds[];
  const int u = xcd_remap(blockIdx.x, p.total_units);
  if (u >= p.total_units) return;
  const int nbh = p.B * p.Hkv;
  const int chunk = u / nbh, bh = u % nbh;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  if (chunk < p.grid_blocks)
    cold_unit<D, KK, KV>(p, b, h, chunk, lds);
  else
    tail_unit<D>(p, b, h, chunk - p.grid_blocks, lds);
}

// Log-sum-exp merge of the partial records of one (sequence, KV head).
template <int D>
__global__ __launch_bounds__(256) void decode_combine_kernel(DecodeParams p) {
  constexpr int PREC = Geo<D>::PREC;
  const int bh = blockIdx.x;
  const int b = bh / p.Hkv, h = bh % p.Hkv;
  for (int idx = threadIdx.x; idx < p.nrep * D; idx += blockDim.x) {
    const int hh = idx / D, d = idx % D;
    float M = -INFINITY;
    for (int u = 0; u < p.units_per_bh; ++u) M = fmaxf(M, record_ptr(p, b, h, u, hh, PREC)[0]);
    float L = 0.f, O = 0.f;
    if (M != -INFINITY) {
      for (int u = 0; u < p.units_per_bh; ++u) {
        const float* r = record_ptr(p, b, h, u, hh, PREC);
        const float m = r[0];
        if (m == -INFINITY) continue;
        const float a = exp2f(m - M);
        L += a * r[1];
        O += a * r[2 + d];
      }
    }
    p.out[b * p.out_sb + (long)(h * p.nrep + hh) * p.out_sh + d] = (h16)(O / L);
  }
}

bool padded_rank_ok(int kp) { return kp == 16 || kp == 32 || kp == 64; }

int fill_params(const ScDecodeArgs* a, DecodeParams* p) {
  if (!a || !a->tier) return sc_fail(SC_ERR_INVALID, "sc_decode_attn: null arguments");
  const ScTierDesc* t = a->tier;
  if (t->head_dim != 64 && t->head_dim != 128)
    return sc_fail(SC_ERR_UNSUPPORTED, "head_dim %d unsupported (64 or 128)", t->head_dim);
  if (!padded_rank_ok(t->kp_keys) || !padded_rank_ok(t->kp_values))
    return sc_fail(SC_ERR_UNSUPPORTED, "padded ranks must be 16, 32 or 64 (got %d, %d)", t->kp_keys, t->kp_values);
  if (t->block_size < 64 || t->block_size % 64)
    return sc_fail(SC_ERR_UNSUPPORTED, "block_size %d must be a positive multiple of 64", t->block_size);
  if (t->batch < 1 || t->kv_heads < 1 || a->q_heads < t->kv_heads || a->q_heads % t->kv_heads)
    return sc_fail(SC_ERR_INVALID, "q_heads %d must be a multiple of kv_heads %d", a->q_heads, t->kv_heads);
  if (a->q_heads / t->kv_heads > kMaxRep)
    return sc_fail(SC_ERR_UNSUPPORTED, "GQA group %d > %d", a->q_heads / t->kv_heads, kMaxRep);
  if (a->grid_blocks < 0 || a->grid_blocks > t->max_blocks)
    return sc_fail(SC_ERR_INVALID, "grid_blocks %d outside [0, max_blocks=%d]", a->grid_blocks, t->max_blocks);
  if (a->grid_tail < 0 || a->grid_tail > t->tail_capacity)
    return sc_fail(SC_ERR_INVALID, "grid_tail %d outside [0, tail_capacity=%d]", a->grid_tail, t->tail_capacity);
  if (a->rope_mode < 0 || a->rope_mode > 2) return sc_fail(SC_ERR_INVALID, "bad rope_mode %d", a->rope_mode);
  if (a->rope_mode != SC_ROPE_NONE && (!a->cos || !a->sin || a->rope_len < 1 || a->rope_stride < t->head_dim))
    return sc_fail(SC_ERR_INVALID, "RoPE tables missing or malformed");
  if (!a->q || !a->out || !t->counters) return sc_fail(SC_ERR_INVALID, "null q/out/counters");
  if (a->grid_blocks > 0 && (!t->codes_k || !t->codes_v || !t->scales_k || !t->scales_v || !t->vnorm ||
                             !t->basis_k || !t->basis_v || !t->block_start))
    return sc_fail(SC_ERR_INVALID, "null cold-tier pointer");
  if (a->grid_tail > 0 && (!t->tail_k || !t->tail_v || !t->tail_pos))
    return sc_fail(SC_ERR_INVALID, "null tail pointer");
  if (((uintptr_t)a->q & 15) || (a->q_stride_h & 7) || (a->q_stride_b & 7))
    return sc_fail(SC_ERR_INVALID, "q must be 16-byte aligned with strides multiple of 8");
  if (a->rope_mode != SC_ROPE_NONE && (((uintptr_t)a->cos & 15) || ((uintptr_t)a->sin & 15) || (a->rope_stride & 7)))
    return sc_fail(SC_ERR_INVALID, "cos/sin must be 16-byte aligned with row stride multiple of 8");
  if (a->mask && ((a->mask_stride_h & 3) || (a->mask_stride_b & 3) || ((uintptr_t)a->mask & 3)))
    return sc_fail(SC_ERR_INVALID, "mask must be 4-byte aligned with strides multiple of 4");
  p->B = t->batch;
  p->Hq = a->q_heads;
  p->Hkv = t->kv_heads;
  p->nrep = a->q_heads / t->kv_heads;
  p->TB = t->block_size;
  p->NB = t->max_blocks;
  p->TCAP = t->tail_capacity;
  p->per_row = t->granularity == SC_QUANT_PER_ROW;
  p->rope_mode = a->rope_mode;
  p->rope_len = a->rope_len;
  p->halves_equal = a->halves_equal;
  p->grid_blocks = a->grid_blocks;
  p->tail_units = (a->grid_tail + kTailUnit - 1) / kTailUnit;
  p->units_per_bh = p->grid_blocks + p->tail_units;
  p->total_units = p->units_per_bh * p->B * p->Hkv;
  p->scale = a->scale;
  p->scale_log2 = a->scale * 1.4426950408889634f;
  p->q = (const h16*)a->q;
  p->q_sb = a->q_stride_b;
  p->q_sh = a->q_stride_h;
  p->codes_k = t->codes_k;
  p->codes_v = t->codes_v;
  p->scales_k = t->scales_k;
  p->scales_v = t->scales_v;
  p->vnorm = t->vnorm;
  p->basis_k = (const h16*)t->basis_k;
  p->basis_v = (const h16*)t->basis_v;
  p->block_start = t->block_start;
  p->tail_k = (const h16*)t->tail_k;
  p->tail_v = (const h16*)t->tail_v;
  p->tail_pos = t->tail_pos;
  p->counters = t->counters;
  p->cos = (const h16*)a->cos;
  p->sin = (const h16*)a->sin;
  p->rope_stride = a->rope_stride;
  p->qpos = a->query_pos;
  p->qpos_scalar = a->query_pos_scalar;
  p->mask = a->mask;
  p->mask_sb = a->mask_stride_b;
  p->mask_sh = a->mask_stride_h;
  p->logits = a->logits_out;
  p->lg_sb = a->logits_stride_b;
  p->lg_sh = a->logits_stride_h;
  p->out = (h16*)a->out;
  p->out_sb = a->out_stride_b;
  p->out_sh = a->out_stride_h;
  return SC_OK;
}

size_t workspace_bytes(const DecodeParams& p, int D) {
  return (size_t)p.B * p.Hkv * p.units_per_bh * p.nrep * (D + 2) * sizeof(float);
}

template <int D, int KK, int KV>
int launch(DecodeParams& p, hipStream_t s) {
  const int grid = xcd_grid(p.total_units);
  const size_t cold_lds = (size_t)(2 * kWaves * p.nrep + kWaves * p.nrep * KV + p.nrep * KV + 2 * p.nrep) * 4;
  const size_t tail_lds = (size_t)(2 * kWaves * p.nrep + kWaves * p.nrep * D) * 4;
  const size_t lds = cold_lds > tail_lds ? cold_lds : tail_lds;
  if (grid > 0) {
    hipLaunchKernelGGL((decode_partial_kernel<D, KK, KV>), dim3(grid), dim3(kThreads), lds, s, p);
    int rc = sc_launch_status("decode_partial_kernel");
    if (rc) return rc;
  }
  hipLaunchKernelGGL((decode_combine_kernel<D>), dim3(p.B * p.Hkv), dim3(256), 0, s, p);
  return sc_launch_status("decode_combine_kernel");
}

template <int D, int KK>
int dispatch_kv(DecodeParams& p, int kv, hipStream_t s) {
  switch (kv) {
    case 16: return launch<D, KK, 16>(p, s);
    case 32: return launch<D, KK, 32>(p, s);
    default: return launch<D, KK, 64>(p, s);
  }
}

template <int D>
int dispatch_kk(DecodeParams& p, int kk, int kv, hipStream_t s) {
  switch (kk) {
    case 16: return dispatch_kv<D, 16>(p, kv, s);
    case 32: return dispatch_kv<D, 32>(p, kv, s);
    default: return dispatch_kv<D, 64>(p, kv, s);
  }
}

}  // namespace

extern "C" int sc_decode_workspace_size(const ScDecodeArgs* args, size_t* bytes) {
  DecodeParams p;
  int rc = fill_params(args, &p);
  if (rc) return rc;
  if (!bytes) return sc_fail(SC_ERR_INVALID, "null bytes");
  *bytes = workspace_bytes(p, args->tier->head_dim);
  return SC_OK;
}

extern "C" int sc_decode_attn(const ScDecodeArgs* args, void* workspace, size_t workspace_bytes_, void* stream) {
  DecodeParams p;
  int rc = fill_params(args, &p);
  if (rc) return rc;
  const int D = args->tier->head_dim;
  const size_t need = workspace_bytes(p, D);
  if (!workspace || workspace_bytes_ < need)
    return sc_fail(SC_ERR_WORKSPACE, "decode workspace too small: %zu < %zu bytes", workspace_bytes_, need);
  if (p.units_per_bh == 0) return sc_fail(SC_ERR_INVALID, "empty cache: no blocks and no tail scanned");
  p.ws = (float*)workspace;
  hipStream_t s = (hipStream_t)stream;
  const int kk = args->tier->kp_keys, kv = args->tier->kp_values;
  if (D == 128) return dispatch_kk<128>(p, kk, kv, s);
  return dispatch_kk<64>(p, kk, kv, s);
}
