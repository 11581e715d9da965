// Spectral prefill attention (gfx950): a chunk of query tokens attends over
// every tier of the cache -- cold blocks (INT8 codes + fp16 bases) and the
// FP16 tail -- with a causal mask, without materialising the keys and
// values (the reference's prefill path reconstructs them all with get_kv
// and runs dense attention, integration.py:292-346; keys are rotated at
// their absolute positions with apply_rope, spectral_attention.py:80-114,
// which uses the first half of the cos/sin rows for both halves).
//
// Workgroup = (sequence b, KV head h, 48 or 32 query tokens); its four waves
// are the four query heads of h (GQA group of 4), each over three 16-query
// sub-tiles at padded ranks 16/16, 32/16 and 16/32 and two otherwise, so every
// reconstructed key tile serves 192 or 128 (query, head) pairs.  Per
// 16-token key tile:
//   * cold block: the waves reconstruct K^T = B_K . C^T on MFMA from the
//     INT8 codes (coefficients fp16(code * scale), as the reference stores
//     them), two 16-row d tiles each (d and d + 64, so every RoPE pair is
//     in one wave), round to fp16, rotate, and write K[tok][d] to LDS;
//     tail: the rows come from the FP16 ring and are rotated the same way;
//   * each wave forms S^T = K . Q^T (16 keys x its 16 queries) on MFMA,
//     rounds it like the reference (fp16 scores, then fp16 after the
//     scaling), masks keys after the query's position, and folds the tile
//     into an online softmax (fp32, base e);
//   * values: cold blocks accumulate O_k^T += C_V^T . P^T in rank space and
//     project O_d^T += B_V^T . O_k^T once per block (hi/lo fp16 split of
//     O_k); tail tiles add V^T . P^T directly, V^T read from LDS with
//     transposing reads.
// MFMA 16x16 layouts: output lane (g, n) holds D[4g + j][n]; operand lane
// (g, n) supplies row/column n and the K slots of group g.
#include "sc_common.h"

namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;
// 16-query sub-tiles per wave, by padded key / value rank (8192-token
// prompt, 16 cold blocks, same-process timings against two sub-tiles):
// three at 16/16, 32/16 and 16/32, with the cold-tile inputs fetched one
// tile ahead instead of two (6, 12 and 22 spilled VGPRs): 1.231 -> 1.045,
// 1.231 -> 1.080 and 1.356 -> 1.168 ms.  With inputs two tiles ahead three
// sub-tiles spill 14, 20 and 31 (1.113, 1.132 and 1.558 ms).  Two at the
// larger ranks (no spills); four spill 116.
constexpr int qs_for(int kk, int kv) { return (kv == 16 && kk <= 32) || (kk == 16 && kv == 32) ? 3 : 2; }
constexpr int kKT = 16;            // key tokens per tile
constexpr int kPitch = 128 + 8;    // LDS row pitch (halves) of a K or V tile
constexpr int kTile = kKT * kPitch;  // halves per LDS tile

struct PrefillParams {
  ScTierDesc t;
  int Hq, Tq, nqt;
  const h16* q;
  long q_sb, q_sh, q_st;
  const int32_t* qpos;  // [B][Tq]
  long qpos_sb;
  const h16* cos;
  const h16* sin;
  long rope_stride;
  int rope_len;
  float scale;
  h16* out;
  long o_sb, o_sh, o_st;
};

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_s4;

// Rotate the (x1, x2) = (K[d], K[d + 64]) pairs of one lane (4 consecutive
// d) with apply_rope's formula in fp16 arithmetic (each product and
// difference rounded, as torch does on fp16 tensors; c, s = the first-half
// cos / sin at the key's position), then store them as K[tok][d] into the
// LDS tile row.
__device__ __forceinline__ void rope_rotate_store(half4_t x1, half4_t x2, half4_t c, half4_t s, int d1, h16* krow) {
  // two packed fp16 pairs per operand: every product and sum rounded to fp16
  typedef h16 half2_v __attribute__((ext_vector_type(2)));
  half4_t o1, o2;
#pragma unroll
  for (int e = 0; e < 4; e += 2) {
    const half2_v X1 = {x1[e], x1[e + 1]}, X2 = {x2[e], x2[e + 1]};
    const half2_v C = {c[e], c[e + 1]}, S = {s[e], s[e + 1]};
    const half2_v a = X1 * C, b = X2 * S, a2 = X2 * C, b2 = X1 * S;
    const half2_v r1 = a - b, r2 = a2 + b2;
    o1[e] = r1.x;
    o1[e + 1] = r1.y;
    o2[e] = r2.x;
    o2[e + 1] = r2.y;
  }
  *reinterpret_cast<half4_t*>(krow + d1) = o1;
  *reinterpret_cast<half4_t*>(krow + d1 + 64) = o2;
}

// cos / sin (first half) at position pos, columns d1 .. d1 + 3; the row is
// clamped into the table (the host cannot see positions).
__device__ __forceinline__ void rope_rows(const PrefillParams& p, int pos, int d1, half4_t& c, half4_t& s) {
  const long row = min(max(pos, 0), p.rope_len - 1);
  c = *reinterpret_cast<const half4_t*>(p.cos + row * p.rope_stride + d1);
  s = *reinterpret_cast<const half4_t*>(p.sin + row * p.rope_stride + d1);
}

template <int KK, int KV>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void prefill_kernel(PrefillParams p) {
  __shared__ __align__(16) h16 kbuf[2][kTile];
  __shared__ __align__(16) h16 vbuf[2][kTile];
  const ScTierDesc& t = p.t;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int w = threadIdx.x >> 6;
  // Causal work grows with the query tile: workgroups are dispatched
  // heaviest first (last query tile of every (sequence, head) first), so
  // the light ones fill in at the end instead of a heavy one trailing.
  constexpr int kQS = qs_for(KK, KV);
  constexpr int kQT = 16 * kQS;
  constexpr bool kShallow = kQS == 3;  // cold-tile inputs one tile ahead (fewer live registers)
  const int nbh = p.t.batch * p.t.kv_heads;
  const int qt = p.nqt - 1 - (int)(blockIdx.x / nbh);
  const int bh = blockIdx.x % nbh;
  const int b = bh / t.kv_heads, h = bh % t.kv_heads;
  const int qh = h * 4 + w;
  const int q0 = qt * kQT;
  int qi[kQS], qpos[kQS];  // this lane's query column in each sub-tile
  bool qvalid[kQS];
  // largest query position of the workgroup (keys beyond it are skipped)
  int qmax = -1;
#pragma unroll
  for (int u = 0; u < kQS; ++u) {
    qi[u] = q0 + 16 * u + n;
    qvalid[u] = qi[u] < p.Tq;
    qpos[u] = qvalid[u] ? p.qpos[b * p.qpos_sb + qi[u]] : -1;
    qmax = max(qmax, qpos[u]);
  }
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) qmax = max(qmax, __shfl_xor(qmax, o));
  // smallest query position of each sub-tile (-1 if a query is past t_q):
  // key tiles entirely at or before it need no mask
  int qmin[kQS];
#pragma unroll
  for (int u = 0; u < kQS; ++u) {
    qmin[u] = qpos[u];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) qmin[u] = min(qmin[u], __shfl_xor(qmin[u], o));
  }
  // Q^T operands: lane (g, n) supplies Q[q n of sub-tile u][32 s + 8 g .. +7]
  half8_t qb[kQS][4];
#pragma unroll
  for (int u = 0; u < kQS; ++u) {
    const h16* qr = p.q + b * p.q_sb + (long)qh * p.q_sh + (long)(qvalid[u] ? qi[u] : 0) * p.q_st;
#pragma unroll
    for (int s = 0; s < 4; ++s)
      qb[u][s] = qvalid[u] ? *reinterpret_cast<const half8_t*>(qr + 32 * s + 8 * g) : (half8_t)(h16)0;
  }
  constexpr int NTV = KV / 16;
  float m[kQS], l[kQS];
  float4_t od[kQS][8], ok[kQS][NTV];
#pragma unroll
  for (int u = 0; u < kQS; ++u) {
    m[u] = -INFINITY;
    l[u] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) od[u][i] = (float4_t)0.f;
#pragma unroll
    for (int i = 0; i < NTV; ++i) ok[u][i] = (float4_t)0.f;
  }
  const int32_t* cnt = t.counters + b * SC_NCOUNTERS;
  const int ncold = cnt[SC_CNT_NCOLD];
  const bool per_row = t.granularity == SC_QUANT_PER_ROW;
  int buf = 0;

  // Scores of the tile in kbuf[buf] against each query sub-tile, masked,
  // folded into the sub-tile's softmax state; pp[u] = P^T (lane (g, n):
  // P[tok 4g + j][q n of sub-tile u]) as fp16.
  // kmax: largest key position of the tile (INT_MAX when unknown: always masked).
  auto scores = [&](const int (&kpos)[4], int kmax, half4_t (&pp)[kQS]) __attribute__((always_inline)) {
    const h16* kr = kbuf[buf] + n * kPitch;
    half8_t ka[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ka[s] = *reinterpret_cast<const half8_t*>(kr + 32 * s + 8 * g);
#pragma unroll
    for (int u = 0; u < kQS; ++u) {
      float4_t sacc = (float4_t)0.f;
#pragma unroll
      for (int s = 0; s < 4; ++s) sacc = mfma_16x16x32(ka[s], qb[u][s], sacc);
      float sv[4];
      float tmax = -INFINITY;
      const bool visible = kmax <= qmin[u];  // wave-uniform: every key before every query
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // reference rounding: fp16 matmul output, then fp16 after the scaling
        const float s16 = (float)(h16)sacc[j];
        float v = (float)(h16)(s16 * p.scale);
        if (!visible && (!qvalid[u] || kpos[j] < 0 || kpos[j] > qpos[u])) v = -INFINITY;
        sv[j] = v;
        tmax = fmaxf(tmax, v);
      }
      tmax = max_over_rows(tmax);
      const float mn = fmaxf(m[u], tmax);
      pp[u] = (half4_t)(h16)0;
      if (mn != -INFINITY) {
        // base 2: exp(x - mn) = exp2(x log2e - mn log2e); masked scores (-inf)
        // and the first tile's m = -inf give exp2(-inf) = 0.  Where the maximum
        // did not grow the factor is set to 1: the fused form would be
        // exp2 of the rounding error of m log2e (1 +- 2^-23 for |m log2e| >= 2),
        // which rescaled l on every tile, fully masked ones included, and not
        // the accumulators, so results drifted with the number of key tiles
        // a query passed through.
        const float mnl = mn * kLog2e;
        const float alpha = mn > m[u] ? __builtin_amdgcn_exp2f(__builtin_fmaf(m[u], kLog2e, -mnl)) : 1.f;
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], kLog2e, -mnl));
          pp[u][j] = (h16)e;
          ls += e;
        }
        l[u] = l[u] * alpha + sum_over_rows(ls);
        // alpha is exactly 1 where the maximum did not grow: the accumulators
        // are rescaled only when some query of the wave saw a larger score
        if (__any(mn > m[u])) {
#pragma unroll
          for (int i = 0; i < 8; ++i) od[u][i] *= alpha;
#pragma unroll
          for (int i = 0; i < NTV; ++i) ok[u][i] *= alpha;
        }
        m[u] = mn;
      }
    }
  };

  // ---------------------------------------------------------------- cold blocks
  for (int j = 0; j < ncold; ++j) {
    const int start = t.block_start[(long)b * t.max_blocks + j];
    if (start > qmax) continue;  // the whole block is after every query
    const long bhj = ((long)b * t.kv_heads + h) * t.max_blocks + j;
    const int8_t* ck = t.codes_k + bhj * t.block_size * KK;
    const int8_t* cv = t.codes_v + bhj * KV * t.block_size;
    const float* sk = t.scales_k + (per_row ? bhj * t.block_size : bhj);
    const float* svp = t.scales_v + (per_row ? bhj * t.block_size : bhj);
    const h16* bk = (const h16*)t.basis_k + bhj * 128 * KK;
    const h16* bv = (const h16*)t.basis_v + bhj * 128 * KV;
    // A operands of this wave's two d tiles: basis rows d = 16 mt + n, mt in {w, w + 4}
    constexpr int KC = KK >= 32 ? KK / 32 : 1;
    half8_t ak[2][KC];
    half4_t ak4[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const h16* row = bk + (long)(16 * (w + 4 * u) + n) * KK;
      if constexpr (KK == 16) {
        ak4[u] = *reinterpret_cast<const half4_t*>(row + 4 * g);
      } else {
#pragma unroll
        for (int c = 0; c < KC; ++c) ak[u][c] = *reinterpret_cast<const half8_t*>(row + 32 * c + 8 * g);
      }
    }
    // tiles that hold a key at or before the last query of the workgroup
    const int ntl = min(t.block_size / kKT, (qmax - start) / kKT + 1);
    // Global inputs of one tile (loaded ahead of their use, see below).
    struct TileIn {
      uint2 ck[KC];   // K codes of token tok0 + n (KK = 16: 4 bytes in .x)
      float scl;      // its K scale
      half4_t c, s;   // cos / sin (first half) at its position, columns d1 .. d1 + 3
      uint32_t cv[NTV];  // V codes of tokens tok0 + 4g .. +3, rank 16 nt + n
      float4_t sv4;   // V scales of those tokens
    };
    const int d1 = 16 * w + 4 * g;
    auto load_in = [&](int tok0, TileIn& in) __attribute__((always_inline)) {
      const int tok = tok0 + n;
      if constexpr (KK == 16) {
        in.ck[0].x = *reinterpret_cast<const uint32_t*>(ck + (long)tok * KK + 4 * g);
      } else {
#pragma unroll
        for (int c = 0; c < KC; ++c) in.ck[c] = *reinterpret_cast<const uint2*>(ck + (long)tok * KK + 32 * c + 8 * g);
      }
      in.scl = per_row ? sk[tok] : sk[0];
      rope_rows(p, start + tok, d1, in.c, in.s);
#pragma unroll
      for (int nt = 0; nt < NTV; ++nt)
        in.cv[nt] = *reinterpret_cast<const uint32_t*>(cv + (long)(16 * nt + n) * t.block_size + tok0 + 4 * g);
      in.sv4 = per_row ? *reinterpret_cast<const float4_t*>(svp + tok0 + 4 * g) : (float4_t)svp[0];
    };
    // Reconstruct + rotate the tile whose inputs are in `in` into kbuf[slot].
    auto recon = [&](const TileIn& in, int slot) __attribute__((always_inline)) {
      float4_t x[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) x[u] = (float4_t)0.f;
      if constexpr (KK == 16) {
        half4_t cf;
#pragma unroll
        for (int e = 0; e < 4; ++e) cf[e] = (h16)((float)(int8_t)(in.ck[0].x >> (8 * e)) * in.scl);
#pragma unroll
        for (int u = 0; u < 2; ++u) x[u] = mfma_16x16x16(ak4[u], cf, x[u]);
      } else {
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          half8_t cf;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            cf[e] = (h16)((float)(int8_t)(in.ck[c].x >> (8 * e)) * in.scl);
            cf[4 + e] = (h16)((float)(int8_t)(in.ck[c].y >> (8 * e)) * in.scl);
          }
#pragma unroll
          for (int u = 0; u < 2; ++u) x[u] = mfma_16x16x32(ak[u][c], cf, x[u]);
        }
      }
      // lane (g, n) holds K[tok n][16 mt + 4 g + j]: x[0] is d1 = 16 w + 4 g, x[1] is d1 + 64
      half4_t x1, x2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x1[e] = (h16)x[0][e];
        x2[e] = (h16)x[1][e];
      }
      rope_rotate_store(x1, x2, in.c, in.s, d1, kbuf[slot] + n * kPitch);
    };
    // Software pipeline over the tiles: tile tt + 1 is reconstructed into
    // the other LDS buffer before tile tt's scores and values (independent
    // work the scheduler can interleave), with one barrier per tile; the
    // global inputs run two tiles ahead of their reconstruction.  With
    // kShallow they run one tile ahead: tile tt + 1's loads are issued
    // before tile tt's scores, which cover their latency, and the tile is
    // reconstructed after them (one set of inputs fewer in registers).
    TileIn cur, nxt, nx2;
    load_in(0, cur);
    if (!kShallow && ntl > 1) load_in(kKT, nxt);
    recon(cur, buf);
    __syncthreads();
    for (int tt = 0; tt < ntl; ++tt) {
      const int tok0 = tt * kKT;
      if constexpr (kShallow) {
        if (tt + 1 < ntl) load_in(tok0 + kKT, nxt);
      } else {
        if (tt + 2 < ntl) load_in(tok0 + 2 * kKT, nx2);
        if (tt + 1 < ntl) recon(nxt, buf ^ 1);
      }
      int kpos[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) kpos[e] = start + tok0 + 4 * g + e;
      half4_t pp[kQS];
      scores(kpos, start + tok0 + kKT - 1, pp);
      if constexpr (kShallow) {
        if (tt + 1 < ntl) recon(nxt, buf ^ 1);
      }
      // ---- values in rank space: O_k^T[16 nt + n][q] += C_V[tok 4g + e][16 nt + n] * P[tok][q]
#pragma unroll
      for (int nt = 0; nt < NTV; ++nt) {
        half4_t a;
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = (h16)((float)(int8_t)(cur.cv[nt] >> (8 * e)) * cur.sv4[e]);
#pragma unroll
        for (int u = 0; u < kQS; ++u) ok[u][nt] = mfma_16x16x16(a, pp[u], ok[u][nt]);
      }
      __syncthreads();  // tile tt read by every wave; tile tt + 1 written
      buf ^= 1;
      cur = nxt;
      if constexpr (!kShallow) nxt = nx2;
    }
    // ---- projection of the block: O_d^T[d][q] += B_V[d][k] O_k^T[k][q] (hi + lo fp16 parts)
    half4_t ph[kQS][NTV], pl[kQS][NTV];
#pragma unroll
    for (int u = 0; u < kQS; ++u)
#pragma unroll
      for (int nt = 0; nt < NTV; ++nt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const h16 hi = (h16)ok[u][nt][e];
          ph[u][nt][e] = hi;
          pl[u][nt][e] = (h16)(ok[u][nt][e] - (float)hi);
        }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int nt = 0; nt < NTV; ++nt) {
        const half4_t a = *reinterpret_cast<const half4_t*>(bv + (long)(16 * mt + n) * KV + 16 * nt + 4 * g);
#pragma unroll
        for (int u = 0; u < kQS; ++u) {
          od[u][mt] = mfma_16x16x16(a, ph[u][nt], od[u][mt]);
          od[u][mt] = mfma_16x16x16(a, pl[u][nt], od[u][mt]);
        }
      }
#pragma unroll
    for (int u = 0; u < kQS; ++u)
#pragma unroll
      for (int i = 0; i < NTV; ++i) ok[u][i] = (float4_t)0.f;
  }

  // ---------------------------------------------------------------- FP16 tail
  const int tl = cnt[SC_CNT_TAIL_LEN], thead = cnt[SC_CNT_TAIL_HEAD];
  const h16* tk = (const h16*)t.tail_k + ((long)b * t.kv_heads + h) * t.tail_capacity * 128;
  const h16* tv = (const h16*)t.tail_v + ((long)b * t.kv_heads + h) * t.tail_capacity * 128;
  const int32_t* tp = t.tail_pos + (long)b * t.tail_capacity;
  // Global inputs of one tail tile, loaded a tile ahead of their use: lane
  // (g, n) takes token tok0 + n, columns d1 .. d1 + 3 and d1 + 64 .. of K
  // and V, and the positions of tokens tok0 + 4g .. +3 (the mask).
  struct TailIn {
    half4_t x1, x2, v1, v2, c, s;
    int kpos[4];
  };
  const int td1 = 16 * w + 4 * g;
  // Ring slot of tail token i < tl: head < capacity and tl <= capacity, so
  // one conditional subtraction replaces the integer modulo; the clamp keeps
  // even inconsistent counters inside the ring.
  auto ring_slot = [&](int i) __attribute__((always_inline)) {
    const int r = thead + i;
    return min(r >= t.tail_capacity ? r - t.tail_capacity : r, t.tail_capacity - 1);
  };
  auto load_tail = [&](int tok0, TailIn& in) __attribute__((always_inline)) {
    const int i = tok0 + n;
    const bool valid = i < tl;
    const int slot = valid ? ring_slot(i) : 0;
    const half4_t z = (half4_t)(h16)0;
    in.x1 = in.x2 = in.v1 = in.v2 = in.c = in.s = z;
    if (valid) {
      in.x1 = *reinterpret_cast<const half4_t*>(tk + (long)slot * 128 + td1);
      in.x2 = *reinterpret_cast<const half4_t*>(tk + (long)slot * 128 + td1 + 64);
      in.v1 = *reinterpret_cast<const half4_t*>(tv + (long)slot * 128 + td1);
      in.v2 = *reinterpret_cast<const half4_t*>(tv + (long)slot * 128 + td1 + 64);
      rope_rows(p, tp[slot], td1, in.c, in.s);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int ii = tok0 + 4 * g + e;
      in.kpos[e] = ii < tl ? tp[ring_slot(ii)] : -1;
    }
  };
  TailIn tcur, tnxt;
  if (tl > 0) load_tail(0, tcur);
  for (int tok0 = 0; tok0 < tl; tok0 += kKT) {
    if (tok0 + kKT < tl) load_tail(tok0 + kKT, tnxt);
    rope_rotate_store(tcur.x1, tcur.x2, tcur.c, tcur.s, td1, kbuf[buf] + n * kPitch);
    *reinterpret_cast<half4_t*>(vbuf[buf] + n * kPitch + td1) = tcur.v1;
    *reinterpret_cast<half4_t*>(vbuf[buf] + n * kPitch + td1 + 64) = tcur.v2;
    __syncthreads();
    half4_t pp[kQS];
    scores(tcur.kpos, 0x7fffffff, pp);
    // O_d^T[16 mt + n][q] += V[tok 4g + e][16 mt + n] P[tok][q]; V^T by transposing reads:
    // lane L of group g addresses row 4g + (L >> 2), columns 16 mt + 4 (L & 3)
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const h16* src = vbuf[buf] + (4 * g + (n >> 2)) * kPitch + 16 * mt + 4 * (n & 3);
      const short4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)src);
#pragma unroll
      for (int u = 0; u < kQS; ++u) od[u][mt] = mfma_16x16x16(__builtin_bit_cast(half4_t, r), pp[u], od[u][mt]);
    }
    buf ^= 1;
    tcur = tnxt;
  }

  // ---------------------------------------------------------------- output
#pragma unroll
  for (int u = 0; u < kQS; ++u) {
    if (qvalid[u]) {
      const float il = l[u] > 0.f ? 1.f / l[u] : 0.f;
      h16* o = p.out + b * p.o_sb + (long)qh * p.o_sh + (long)qi[u] * p.o_st;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        half4_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (h16)(od[u][mt][e] * il);
        *reinterpret_cast<half4_t*>(o + 16 * mt + 4 * g) = v;
      }
    }
  }
}

template <int KK>
int launch_kv(const PrefillParams& p, int kv, dim3 grid, hipStream_t s) {
  switch (kv) {
    case 16: hipLaunchKernelGGL((prefill_kernel<KK, 16>), grid, dim3(kThreads), 0, s, p); break;
    case 32: hipLaunchKernelGGL((prefill_kernel<KK, 32>), grid, dim3(kThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((prefill_kernel<KK, 64>), grid, dim3(kThreads), 0, s, p); break;
  }
  return sc_launch_status("prefill_kernel");
}

}  // namespace

extern "C" int sc_prefill_attn(const ScPrefillArgs* a, void* stream) {
  if (!a || !a->tier) return sc_fail(SC_ERR_INVALID, "sc_prefill_attn: null arguments");
  const ScTierDesc* t = a->tier;
  if (t->head_dim != 128) return sc_fail(SC_ERR_UNSUPPORTED, "prefill: head_dim %d unsupported (128)", t->head_dim);
  if (a->q_heads != 4 * t->kv_heads)
    return sc_fail(SC_ERR_UNSUPPORTED, "prefill: GQA group %d unsupported (4 query heads per KV head)",
                   t->kv_heads ? a->q_heads / t->kv_heads : 0);
  const int kk = t->kp_keys, kv = t->kp_values;
  if ((kk != 16 && kk != 32 && kk != 64) || (kv != 16 && kv != 32 && kv != 64))
    return sc_fail(SC_ERR_UNSUPPORTED, "prefill: padded ranks must be 16, 32 or 64 (got %d, %d)", kk, kv);
  if (t->block_size < kKT || t->block_size % kKT)
    return sc_fail(SC_ERR_UNSUPPORTED, "prefill: block_size %d must be a multiple of %d", t->block_size, kKT);
  if (a->t_q < 0) return sc_fail(SC_ERR_INVALID, "prefill: t_q %d < 0", a->t_q);
  if (a->rope_len < 1) return sc_fail(SC_ERR_INVALID, "prefill: empty RoPE tables");
  if (!a->q || !a->out || !a->query_pos || !a->cos || !a->sin)
    return sc_fail(SC_ERR_INVALID, "prefill: null q / out / query_pos / cos / sin");
  if (((uintptr_t)a->q & 15) || (a->q_stride_t % 8) || (a->q_stride_h % 8) || (a->q_stride_b % 8) ||
      ((uintptr_t)a->out & 7) || (a->out_stride_t % 4) || ((uintptr_t)a->cos & 7) || ((uintptr_t)a->sin & 7) ||
      (a->rope_stride % 4))
    return sc_fail(SC_ERR_INVALID, "prefill: misaligned q / out / RoPE tables");
  if (a->t_q == 0) return SC_OK;
  PrefillParams p;
  p.t = *t;
  p.Hq = a->q_heads;
  p.Tq = a->t_q;
  const int qt_tokens = 16 * qs_for(kk, kv);
  p.nqt = (a->t_q + qt_tokens - 1) / qt_tokens;
  p.q = (const h16*)a->q;
  p.q_sb = a->q_stride_b;
  p.q_sh = a->q_stride_h;
  p.q_st = a->q_stride_t;
  p.qpos = a->query_pos;
  p.qpos_sb = a->query_pos_stride_b;
  p.cos = (const h16*)a->cos;
  p.sin = (const h16*)a->sin;
  p.rope_stride = a->rope_stride;
  p.rope_len = a->rope_len;
  p.scale = a->scale;
  p.out = (h16*)a->out;
  p.o_sb = a->out_stride_b;
  p.o_sh = a->out_stride_h;
  p.o_st = a->out_stride_t;
  const long nwg = (long)t->batch * t->kv_heads * p.nqt;
  if (nwg > 0x7fffffffL) return sc_fail(SC_ERR_UNSUPPORTED, "prefill: grid too large");
  const dim3 grid((unsigned)nwg);
  hipStream_t s = (hipStream_t)stream;
  switch (kk) {
    case 16: return launch_kv<16>(p, kv, grid, s);
    case 32: return launch_kv<32>(p, kv, grid, s);
    default: return launch_kv<64>(p, kv, grid, s);
  }
}
