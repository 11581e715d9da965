// Decode attention over the three-tier spectral cache (gfx950).
//
// Replaces the per-block PyTorch loops of
//   spectral_attention_decode   kernels/spectral_attention.py:684-857 (absolute RoPE)
//   spectral_attention_forward  spectral_attention.py:117-349          (distance RoPE)
// with one split-K kernel plus a log-sum-exp combine.
//
// Work unit = (sequence b, group of four KV heads hq, unit j); one
// 256-thread workgroup whose wave w owns KV head 4 hq + w and its GQA group
// of query heads.  Unit j walks cold block j / split (or its share of the
// block when a block is split over `split` workgroups) in ranges of 64
// tokens, then folds in FP16 tail tiles j, j + W, ... (16 tokens each; W
// units per (sequence, head group)).  Each wave writes one
// partial record (running max, sum, unnormalised output) per query head;
// decode_combine_kernel merges the records of a (sequence, query head).
//
// Per range and wave (phases of consecutive ranges overlap: phase C of
// range r - 1 runs after phase A of range r):
//   A. per 16-token tile: X^T = B_K^T . code^T on MFMA (codes -> fp16
//      exactly in registers; basis rows permuted so that a lane holds the
//      RoPE pairs (d, d + D/2) of one token), RoPE of the reconstructed key
//      in packed fp16 with the cos/sin rows staged in LDS (phi = p, or
//      max(q - p, 0) in distance mode), scores of the GQA group
//      S = Y . Q^T on MFMA, times the row scale, rounded at the reference's
//      fp16 cast points; the next range's codes are loaded meanwhile;
//   B. the range maximum merged into the running maximum (base 2);
//   C. per tile: P = exp2(logit - max), Pacc^T += C_V^T . (P * s_V) on MFMA.
// Token order inside a 64-token range is permuted (lane group g of a score
// tile holds tokens 16g + 4i + j of tile i) so that the V codes of four
// tiles are one 16-byte load per lane and per-row scales are one coalesced
// load per 64 tokens.  After the last range, Pacc is projected once through
// B_V (d-major) and added to the tail tile's output.
//
// GEN = false is the branch-free path (RoPE absolute or distance over an
// HF table whose halves are equal, no mask, no logits output); GEN = true
// adds the keep-mask, the logits output, unequal table halves and
// rope_mode = none.
#include <math.h>

#include <atomic>
#include <type_traits>

#include "sc_common.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 16;
constexpr int kMaxRep = 16;
constexpr long kFillUnits = 256;  // a split grid stops at one workgroup per CU (256 CUs)
// A CU's wave arbiter favours its oldest waves: of two resident workgroups,
// the one dispatched second runs at about half the speed of the first and
// finishes ~8 us after it (batch 8, 16K context).  It raises its priority
// once it has finished this many ranges, which evens out the finish times.
constexpr int kYoungPrioRange = 2;
constexpr int kVRow = 132;                              // LDS row (halves) of a staged V tile
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeParams {
  int B, Hq, Hkv, nrep, TB, NB, TCAP, per_row, rope_mode, rope_len, halves_equal;
  int grid_blocks, tpw, n_hq, cold_units, units_per_bh, fold_tail;
  int split;  // workgroups per cold block (each takes TB / (64 * split) consecutive ranges)
  int young_slot;  // slots (blockIdx / 8) from here on were dispatched after every CU had a workgroup
  long n_cold_units;  // summed over (b, head group)
  float scale;
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
  int qpos_scalar, qpos64;  // qpos64: qpos points to int64 positions
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
// With equal halves (c1 = c2, s1 = s2) all three are (c x1 - s x2, s x1 + c x2).
enum RotKind { kRotColdAbs = 0, kRotTailAbs = 1, kRotDist = 2 };

template <int D>
struct Geo {
  static constexpr int HALF = D / 2;
  static constexpr int QG = HALF / 4;  // RoPE pairs per lane
  static constexpr int NV = QG / 8;    // half8 vectors per lane and half
  static constexpr int MT = D / 16;    // 16-row tiles over d
  static constexpr int MTH = MT / 2;
  static constexpr int DS = D / 32;    // K-steps of the score MFMA (= 2 NV)
  static constexpr int PREC = D + 4;   // partial record: m, l, -, -, o[D] (o 16-byte aligned)
};

template <int NV>
struct Half8s {
  half8_t v[NV];
};

template <int NV>
__device__ __forceinline__ Half8s<NV> load_h8s(const h16* src) {
  Half8s<NV> r;
#pragma unroll
  for (int i = 0; i < NV; ++i) r.v[i] = *reinterpret_cast<const half8_t*>(src + 8 * i);
  return r;
}

// Packs the reconstruct MFMA outputs of one lane into the x1 / x2 halves:
// x1 element 4*mt + j = x[mt][j] (mt < MTH), x2 from x[MTH + mt].
template <int D>
__device__ __forceinline__ void pack_x(const float4_t (&x)[Geo<D>::MT], Half8s<Geo<D>::NV>& x1,
                                       Half8s<Geo<D>::NV>& x2) {
  using G = Geo<D>;
#pragma unroll
  for (int v = 0; v < G::NV; ++v) {
    const float4_t a = x[2 * v], b = x[2 * v + 1], c = x[G::MTH + 2 * v], d = x[G::MTH + 2 * v + 1];
    x1.v[v] = (half8_t){(h16)a[0], (h16)a[1], (h16)a[2], (h16)a[3], (h16)b[0], (h16)b[1], (h16)b[2], (h16)b[3]};
    x2.v[v] = (half8_t){(h16)c[0], (h16)c[1], (h16)c[2], (h16)c[3], (h16)d[0], (h16)d[1], (h16)d[2], (h16)d[3]};
  }
}

// Rotated key as the A operand of the score MFMA (K-step s < DS/2 -> first
// half, else second half).  c1/s1 are the lane's first-half table entries;
// c2/s2 its second-half entries (== c1/s1 when the halves are equal).
template <int D>
__device__ __forceinline__ void rotate(const Half8s<Geo<D>::NV>& x1, const Half8s<Geo<D>::NV>& x2,
                                       const Half8s<Geo<D>::NV>& c1, const Half8s<Geo<D>::NV>& s1,
                                       const Half8s<Geo<D>::NV>& c2, const Half8s<Geo<D>::NV>& s2, int kind,
                                       half8_t (&ya)[Geo<D>::DS]) {
  using G = Geo<D>;
#pragma unroll
  for (int v = 0; v < G::NV; ++v) {
    const half8_t sa = (kind == kRotColdAbs) ? s2.v[v] : s1.v[v];
    const half8_t sb = (kind == kRotTailAbs) ? s2.v[v] : s1.v[v];
    const half8_t cb = (kind == kRotDist) ? c1.v[v] : c2.v[v];
    ya[v] = c1.v[v] * x1.v[v] - sa * x2.v[v];
    ya[G::NV + v] = sb * x1.v[v] + cb * x2.v[v];
  }
}

template <int D>
__device__ __forceinline__ void rotate_he(const Half8s<Geo<D>::NV>& x1, const Half8s<Geo<D>::NV>& x2,
                                          const Half8s<Geo<D>::NV>& c, const Half8s<Geo<D>::NV>& s,
                                          half8_t (&ya)[Geo<D>::DS]) {
  using G = Geo<D>;
#pragma unroll
  for (int v = 0; v < G::NV; ++v) {
    ya[v] = c.v[v] * x1.v[v] - s.v[v] * x2.v[v];
    ya[G::NV + v] = s.v[v] * x1.v[v] + c.v[v] * x2.v[v];
  }
}

template <int D>
__device__ __forceinline__ void unrotated(const Half8s<Geo<D>::NV>& x1, const Half8s<Geo<D>::NV>& x2,
                                          half8_t (&ya)[Geo<D>::DS]) {
  using G = Geo<D>;
#pragma unroll
  for (int v = 0; v < G::NV; ++v) {
    ya[v] = x1.v[v];
    ya[G::NV + v] = x2.v[v];
  }
}

// Query operand of the score MFMA: lane (g, n) holds query head qh of the
// group (its MFMA column), d-slots of K-step s = the lane group's RoPE
// pairs, matching the Y layout.
template <int D>
__device__ __forceinline__ void load_q(const DecodeParams& p, int b, int h, int g, int qh, half8_t (&qb)[Geo<D>::DS]) {
  using G = Geo<D>;
  const h16* qrow = p.q + b * p.q_sb + (long)(h * p.nrep + qh) * p.q_sh;
#pragma unroll
  for (int s = 0; s < G::DS; ++s) {
    const int d0 = (s < G::NV) ? g * G::QG + 8 * s : G::HALF + g * G::QG + 8 * (s - G::NV);
    qb[s] = *reinterpret_cast<const half8_t*>(qrow + d0);
  }
}

__device__ __forceinline__ float* record_ptr(const DecodeParams& p, int b, int h, int unit, int hh, int prec) {
  return p.ws + ((((long)(b * p.Hkv + h) * p.units_per_bh + unit) * p.nrep + hh) * prec);
}

__device__ __forceinline__ int clamp_angle(int phi, int len) { return min(max(phi, 0), len - 1); }

// The reference rounds scores and logits to the model dtype (fp16) before
// the fp32 softmax: s = fp16(raw) (kernels/spectral_attention.py:446,
// spectral_attention.py:238), logits = fp16(s * scale) (:280-281).
__device__ __forceinline__ h16 fp16_logit(float raw, float scale) {
  return (h16)((float)(h16)raw * scale);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Maximum of a lane's logits (fp16, four per tile) in the log2 domain.
template <int NTILE>
__device__ __forceinline__ float lane_max_log2(const half4_t (&lg)[NTILE]) {
  half4_t m = lg[0];
#pragma unroll
  for (int i = 1; i < NTILE; ++i) m = __builtin_elementwise_max(m, lg[i]);
  const float a = fmaxf((float)m[0], (float)m[1]), c = fmaxf((float)m[2], (float)m[3]);
  return fmaxf(a, c) * kLog2e;
}

// ------------------------------------------------------------------ cold
// Staged RoPE rows.  LDS row rho of a range holds the cos/sin entries of
// range token swap(rho) (bit fields [2:3] and [4:5] exchanged): the 16
// lanes of a score tile then read 16 consecutive rows, and a row pitch of
// an odd number of 16-byte chunks keeps those reads free of bank conflicts.
__device__ __forceinline__ int swap_fields(int r) { return (r & ~0x3c) | ((r & 0x0c) << 2) | ((r & 0x30) >> 2); }

template <int D, bool HE>
struct RopeStage {
  static constexpr int HCH = D / 16;              // 16-byte chunks per half row of one table
  static constexpr int CHT = HE ? HCH : 2 * HCH;  // chunks of one table per staged row
  static constexpr int CH = 2 * CHT;              // cos (1 | 2) then sin (1 | 2)
  static constexpr int ROW = CH * 16 + 16;        // LDS row pitch in bytes
};

// Thread t stages chunk c = k * kThreads + t (k < NS) of each table for a
// range of T rows: staged row c / CHT, table column c % CHT.  The global
// byte offsets are relative to the range's base angle row (the same for
// every range of a block) so that the per-range address is one scalar.
template <int D, bool HE, int T>
struct StageMap {
  static constexpr int NS = T * RopeStage<D, HE>::CHT / kThreads;  // chunks per table per thread
  uint32_t src[NS];  // byte offset of the chunk from the base angle row
  int dst[NS];       // LDS byte offset of the cos chunk (its sin chunk follows CHT chunks later)
};

template <int D, bool HE, int T>
__device__ __forceinline__ StageMap<D, HE, T> stage_map(const DecodeParams& p, bool dist) {
  using RS = RopeStage<D, HE>;
  StageMap<D, HE, T> m;
#pragma unroll
  for (int k = 0; k < StageMap<D, HE, T>::NS; ++k) {
    const int c = k * kThreads + threadIdx.x;
    const int r = c / RS::CHT, col = c % RS::CHT;
    const int tok = swap_fields(r);
    m.src[k] = (uint32_t)(((dist ? T - 1 - tok : tok) * (int)p.rope_stride + 8 * col) * 2);
    m.dst[k] = r * RS::ROW + col * 16;
  }
  return m;
}

// Fetches the RoPE rows of the range starting at token position pos0:
// angle p (absolute) or q - p (distance) of each of its T tokens.  Inside
// the table the range is one contiguous span of rows starting at a
// wave-uniform base; at the table edges each angle is clamped.
template <int N>
struct U4s {
  uint4 v[N];
};

template <int D, bool HE, int T>
__device__ __forceinline__ U4s<2 * StageMap<D, HE, T>::NS> stage_fetch(const DecodeParams& p,
                                                                      const StageMap<D, HE, T>& m, int pos0, int qp,
                                                                      bool dist) {
  using RS = RopeStage<D, HE>;
  constexpr int NS = StageMap<D, HE, T>::NS;
  const int base = dist ? qp - pos0 - (T - 1) : pos0;
  const bool inside = base >= 0 && base + T <= p.rope_len;
  const long b0 = (long)base * p.rope_stride;
  const char* cb = reinterpret_cast<const char*>(p.cos + b0);
  const char* sb = reinterpret_cast<const char*>(p.sin + b0);
  U4s<2 * NS> r;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    if (inside) {
      r.v[k] = *reinterpret_cast<const uint4*>(cb + m.src[k]);
      r.v[NS + k] = *reinterpret_cast<const uint4*>(sb + m.src[k]);
    } else {  // rows at the table edges: clamp each angle
      const int c = k * kThreads + threadIdx.x;
      const int row = c / RS::CHT, col = c % RS::CHT;
      const int pos = pos0 + swap_fields(row);
      const long off = (long)clamp_angle(dist ? max(qp - pos, 0) : pos, p.rope_len) * p.rope_stride + 8 * col;
      r.v[k] = *reinterpret_cast<const uint4*>(p.cos + off);
      r.v[NS + k] = *reinterpret_cast<const uint4*>(p.sin + off);
    }
  }
  return r;
}

template <int D, bool HE, int T>
__device__ __forceinline__ void stage_store(char* buf, const StageMap<D, HE, T>& m,
                                            const U4s<2 * StageMap<D, HE, T>::NS>& v) {
  constexpr int NS = StageMap<D, HE, T>::NS;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    *reinterpret_cast<uint4*>(buf + m.dst[k]) = v.v[k];
    *reinterpret_cast<uint4*>(buf + m.dst[k] + RopeStage<D, HE>::CHT * 16) = v.v[NS + k];
  }
}

template <int D, bool HE>
__device__ __forceinline__ Half8s<Geo<D>::NV> lds_rope(const char* smem, int row, int chunk) {
  Half8s<Geo<D>::NV> r;
#pragma unroll
  for (int v = 0; v < Geo<D>::NV; ++v)
    r.v[v] = *reinterpret_cast<const half8_t*>(smem + row * RopeStage<D, HE>::ROW + (chunk + v) * 16);
  return r;
}

// INT8 codes and scales of one wave's range (16 TPW tokens of one head).
// ONE (one logit per lane): sk[i] / sv[i] hold the row scale of the token
// whose logit the lane holds in tile i.  Otherwise float4: the row scales
// of the four tokens of the lane's score slots (one 16-byte load).
template <int KK, int KV, int TPW, bool ONE>
struct CodeBuf {
  static constexpr int NGRP = TPW / 4, NT = KV / 16, KC = KK >= 32 ? KK / 32 : 1;
  using CodeK = typename std::conditional<KK == 16, uint32_t, uint2>::type;
  using Scale = typename std::conditional<ONE, float, float4_t>::type;
  CodeK kc[TPW][KC];
  uint4 vc[NGRP][NT];
  Scale sk[TPW], sv[TPW];
};

// Sources of one wave's range (range starting at block token tok0).  Each
// part can be issued on its own so that a register is refilled with the
// next range's data right after its last use.
struct CodeSrc {
  const int8_t* ck;   // K codes of the range
  const int8_t* cv;   // V codes of the range
  const float* skp;   // K scales (per row: the range's first token; per head: the value)
  const float* svp;
};

template <int KK, int KV>
__device__ __forceinline__ CodeSrc code_src(const DecodeParams& p, long bhj, int tok0) {
  CodeSrc s;
  s.ck = p.codes_k + bhj * (long)p.TB * KK + (long)tok0 * KK;
  s.cv = p.codes_v + bhj * (long)KV * p.TB + tok0;
  s.skp = p.scales_k + (p.per_row ? bhj * p.TB + tok0 : bhj);
  s.svp = p.scales_v + (p.per_row ? bhj * p.TB + tok0 : bhj);
  return s;
}

// Lane offsets are unsigned 32-bit values added to wave-uniform bases, so
// each load is one SGPR base + VGPR offset (+ immediate) with no per-lane
// 64-bit address arithmetic.
template <int KK, class CB>
__device__ __forceinline__ void load_kc(const CodeSrc& s, int i, CB& cb) {
  const uint32_t lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const uint32_t off = (16 * (n >> 2) + (n & 3)) * KK + (KK == 16 ? 4 : 8) * g;
  const int8_t* base = s.ck + ((i / 4) * 64 + 4 * (i % 4)) * KK;
#pragma unroll
  for (int c = 0; c < CB::KC; ++c) {
    if constexpr (KK == 16)
      cb.kc[i][c] = *reinterpret_cast<const uint32_t*>(base + off);
    else
      cb.kc[i][c] = *reinterpret_cast<const uint2*>(base + c * 32 + off);
  }
}

template <class CB>
__device__ __forceinline__ void load_vc(const DecodeParams& p, const CodeSrc& s, int gr, CB& cb) {
  const uint32_t lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const uint32_t off = n * (uint32_t)p.TB + 16 * g;
#pragma unroll
  for (int nt = 0; nt < CB::NT; ++nt)
    cb.vc[gr][nt] = *reinterpret_cast<const uint4*>(s.cv + (long)nt * 16 * p.TB + gr * 64 + off);
}

// Row scale(s) for tile i of a range: tile i covers range tokens
// 64 (i / 4) + 16 g + 4 (i % 4) + {0..3} in lane group g, and a ONE lane
// holds token ... + (n & 3).  Per head: the block's scale.  PRM: 0 per
// head, 1 per row, 2 decided at run time (general path).
template <int PRM, bool ONE>
__device__ __forceinline__ typename std::conditional<ONE, float, float4_t>::type load_scale(const DecodeParams& p,
                                                                                            const float* base, int i) {
  const uint32_t lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const float* tile = base + 64 * (i / 4) + 4 * (i % 4);
  const bool row = PRM == 1 || (PRM == 2 && p.per_row);
  if constexpr (ONE) {
    return row ? tile[16 * g + (n & 3)] : base[0];
  } else {
    if (row) return *reinterpret_cast<const float4_t*>(tile + 16 * g);
    return (float4_t)base[0];
  }
}

template <int KK, int PRM, bool ONE, class CB>
__device__ __forceinline__ void load_codes(const DecodeParams& p, const CodeSrc& s, CB& cb) {
#pragma unroll
  for (int i = 0; i < CB::NGRP * 4; ++i) load_kc<KK>(s, i, cb);
#pragma unroll
  for (int gr = 0; gr < CB::NGRP; ++gr) load_vc(p, s, gr, cb);
#pragma unroll
  for (int i = 0; i < CB::NGRP * 4; ++i) {
    cb.sk[i] = load_scale<PRM, ONE>(p, s.skp, i);
    cb.sv[i] = load_scale<PRM, ONE>(p, s.svp, i);
  }
}

// Running state of one wave (one KV head) across the ranges of a block.
template <int KV>
struct ColdState {
  float m2, l;  // running max (log2 domain, per head) and lane-partial sum
  float4_t pacc[KV / 16];
};

// Lane roles of the two score layouts.  The score MFMA leaves lane (g, n)
// with tokens 4 g + {0..3} of query column n.
//   ONE = false: column n is query head n (n < nrep); a lane holds four
//                logits, one per token.
//   ONE = true:  column n holds head n >> 2 (each head four times, nrep <= 4)
//                and the lane keeps only token 4 g + (n & 3): one logit per
//                lane, so exp2, scaling and rounding run once per
//                (token, head).  The P operand of P.V is gathered back from
//                the lane's quad (lanes 4 (n >> 2) + {0..3}).
struct Lanes {
  bool b0, b1;    // bits 0 and 1 of n: which of the four tokens a ONE lane keeps
  bool valid;     // ONE: head n >> 2 exists (< nrep); else n < nrep
  uint32_t psel;  // v_perm selector ordering a quad pair by quad-lane index
};
template <bool ONE>
__device__ __forceinline__ Lanes lane_roles(int n, int nrep) {
  Lanes r;
  r.b0 = n & 1;
  r.b1 = (n >> 1) & 1;
  r.valid = ONE ? (n >> 2) < nrep : n < nrep;
  r.psel = (n & 1) ? 0x05040100u : 0x01000504u;
  return r;
}

// P values of the four lanes of this lane's quad, in quad-lane order: the
// fp16 B operand (tokens 4 g + {0..3}) of a 16x16x16 P.V MFMA.  Every lane's
// DPP source lies in its own quad, so the moves leave no lane unwritten and
// their `old` operand is never read: mov_dpp leaves it undefined, which
// saves the zero-initialising move per DPP that update_dpp(0, ...) costs
// here (reductions keep update_dpp: the compiler folds those DPP moves into
// the max/add itself).
__device__ __forceinline__ half4_t quad_gather_h4(float v, uint32_t psel) {
  const uint32_t x = (uint32_t)__builtin_bit_cast(uint16_t, (h16)v);
  const uint32_t y = (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, false);  // lane ^ 1
  const uint32_t pair = __builtin_amdgcn_perm(x, y, psel);  // (even, odd) quad lane of this pair
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)pair, 0x00, 0xF, 0xF, false);  // quad lane 0
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)pair, 0xAA, 0xF, 0xF, false);  // quad lane 2
  return __builtin_bit_cast(half4_t, make_uint2(lo, hi));
}

__device__ __forceinline__ float pick4(const float4_t& v, const Lanes& r) {
  const float a = r.b0 ? v[1] : v[0], c = r.b0 ? v[3] : v[2];
  return r.b1 ? c : a;
}

// Maximum over the lanes holding one query head's logits, in the log2 domain.
template <bool ONE>
__device__ __forceinline__ float head_max(float v) {
  v = max_over_rows(v);
  return ONE ? quad_max(v) : v;
}

// Logits of one range: one per tile (ONE) or four per tile.
template <bool ONE, int TPW>
struct RangeLogits {
  typename std::conditional<ONE, float, half4_t>::type v[TPW];
};

// A range is processed in three phases: scores (A), the range maximum (B)
// and probabilities with P . C_V (C).  Phase C of a range runs in the next
// range's step, after that range's phase A, so that the latency chains of
// C (exp, quad gather, accumulation) overlap A's independent work.

// Phase A: scores of the range's TPW tiles.  If another range follows
// (MORE), its RoPE rows are fetched into registers first and written to the
// other LDS buffer at the end, and each K code and K scale register is
// refilled from nsrc (the next range) right after its last use, so the next
// range's HBM loads are in flight during this one.  MORE and PRM are
// compile-time so that the tile loop has no branches.
template <int D, int KK, int KV, int TPW, bool GEN, bool HE, int PRM, bool MORE, class CB>
__device__ __forceinline__ void range_scores(const DecodeParams& p, CB& cb, const CodeSrc nsrc,
                                             const half8_t (&a8)[Geo<D>::MT][CB::KC],
                                             const half4_t (&a4)[Geo<D>::MT], const half8_t (&qb)[Geo<D>::DS],
                                             const StageMap<D, HE, kTile * TPW>& smap, const char* rope_cur,
                                             char* rope_next, int next_pos0, int qp, bool dist, bool rope,
                                             const uint8_t* mrow, float* lrow, RangeLogits<!GEN, TPW>& lg) {
  using G = Geo<D>;
  using RS = RopeStage<D, HE>;
  constexpr bool ONE = !GEN;
  constexpr int T = kTile * TPW;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const Lanes lr = lane_roles<ONE>(n, p.nrep);
  const bool stage = MORE && rope;
  // The next range's RoPE rows (L2 hits) are requested before any of this
  // range's HBM refills: vmcnt retires in order, so waiting for them before
  // the LDS stores below never waits for the refills.
  U4s<2 * StageMap<D, HE, T>::NS> sv;
  if constexpr (MORE) {
    if (rope)
      sv = stage_fetch<D, HE, T>(p, smap, next_pos0, qp, dist);
    else
      sv = U4s<2 * StageMap<D, HE, T>::NS>{};
  }
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int gr = i / 4, ii = i % 4;
    float4_t x[G::MT];
    if constexpr (KK == 16) {
      const half4_t bc = i8x4_to_h4(cb.kc[i][0]);
      if constexpr (MORE) {
        load_kc<KK>(nsrc, i, cb);
        pin_vmem();
      }
#pragma unroll
      for (int mt = 0; mt < G::MT; ++mt) x[mt] = mfma_16x16x16(a4[mt], bc, (float4_t)0.f);
    } else {
      half8_t bc[CB::KC];
#pragma unroll
      for (int c = 0; c < CB::KC; ++c) bc[c] = i8x8_to_h8(cb.kc[i][c]);
      if constexpr (MORE) {
        load_kc<KK>(nsrc, i, cb);
        pin_vmem();
      }
#pragma unroll
      for (int mt = 0; mt < G::MT; ++mt) {
        float4_t acc = (float4_t)0.f;
#pragma unroll
        for (int c = 0; c < CB::KC; ++c) acc = mfma_16x16x32(a8[mt][c], bc[c], acc);
        x[mt] = acc;
      }
    }
    Half8s<G::NV> x1, x2;
    pack_x<D>(x, x1, x2);
    const int row = gr * 64 + 16 * ii + n;  // staged row of this lane's token
    half8_t ya[G::DS];
    if constexpr (!GEN) {
      rotate_he<D>(x1, x2, lds_rope<D, true>(rope_cur, row, g * G::NV),
                   lds_rope<D, true>(rope_cur, row, RS::HCH + g * G::NV), ya);
    } else {
      if (!rope) {
        unrotated<D>(x1, x2, ya);
      } else if constexpr (HE) {
        rotate_he<D>(x1, x2, lds_rope<D, true>(rope_cur, row, g * G::NV),
                     lds_rope<D, true>(rope_cur, row, RS::HCH + g * G::NV), ya);
      } else {
        // staged row: cos1 | cos2 | sin1 | sin2
        rotate<D>(x1, x2, lds_rope<D, false>(rope_cur, row, g * G::NV),
                  lds_rope<D, false>(rope_cur, row, 2 * RS::HCH + g * G::NV),
                  lds_rope<D, false>(rope_cur, row, RS::HCH + g * G::NV),
                  lds_rope<D, false>(rope_cur, row, 3 * RS::HCH + g * G::NV), dist ? kRotDist : kRotColdAbs, ya);
      }
    }
    float4_t sacc = (float4_t)0.f;
#pragma unroll
    for (int s = 0; s < G::DS; ++s) sacc = mfma_16x16x32(ya[s], qb[s], sacc);
    if constexpr (ONE) {
      const float l = (float)fp16_logit(pick4(sacc, lr) * cb.sk[i], p.scale);
      lg.v[i] = lr.valid ? l : -INFINITY;
      if constexpr (MORE) cb.sk[i] = load_scale<PRM, ONE>(p, nsrc.skp, i);
    } else {
      // lane holds head n, range tokens tg + jj, tg = 64 gr + 16 g + 4 ii
      const int tg = gr * 64 + 16 * g + 4 * ii;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) lg.v[i][jj] = fp16_logit(sacc[jj] * cb.sk[i][jj], p.scale);
      if constexpr (MORE) cb.sk[i] = load_scale<PRM, ONE>(p, nsrc.skp, i);
      if constexpr (GEN) {
        uint32_t keep = 0xffffffffu;
        if (mrow) keep = *reinterpret_cast<const uint32_t*>(mrow + tg);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          if (lrow) lrow[tg + jj] = (float)lg.v[i][jj];
          if (!((keep >> (8 * jj)) & 0xffu)) lg.v[i][jj] = (h16)(-INFINITY);
        }
      }
    }
  }
  if constexpr (MORE) {
    if (stage) stage_store<D, HE, T>(rope_next, smap, sv);
  }
}

// Phase B: the range maximum merged into the running maximum.  Returns the
// subtrahend of the range's exponents (msub) and the rescale of the
// accumulators summed before this range (alpha; applied to the partial sum
// here and to P . C_V in phase C).
template <bool ONE, int TPW, int KV>
__device__ __forceinline__ void range_max(const RangeLogits<ONE, TPW>& lg, ColdState<KV>& st, float& msub,
                                          float& alpha) {
  float mloc;
  if constexpr (ONE) {
    mloc = lg.v[0];
#pragma unroll
    for (int i = 1; i < TPW; ++i) mloc = fmaxf(mloc, lg.v[i]);
    mloc *= kLog2e;
  } else {
    mloc = lane_max_log2<TPW>(lg.v);
  }
  const float mr = head_max<ONE>(mloc);
  const float m_new = fmaxf(st.m2, mr);
  msub = (m_new == -INFINITY) ? 0.f : m_new;
  alpha = fast_exp2(st.m2 - msub);  // exp2(-inf) = 0 on the first range
  st.m2 = m_new;
  st.l *= alpha;
}

// Phase C: probabilities and P . C_V with the V codes and scales in cb.  With
// MORE each V register is refilled from vsrc right after its last use.
template <int KV, int TPW, bool GEN, int PRM, bool MORE, class CB>
__device__ __forceinline__ void range_values(const DecodeParams& p, CB& cb, const CodeSrc vsrc,
                                             const RangeLogits<!GEN, TPW>& lg, float msub, float alpha, float vn,
                                             ColdState<KV>& st) {
  constexpr bool ONE = !GEN;
  const int n = threadIdx.x & 15;
  const Lanes lr = lane_roles<ONE>(n, p.nrep);
#pragma unroll
  for (int nt = 0; nt < CB::NT; ++nt) st.pacc[nt] *= alpha;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int gr = i / 4, ii = i % 4;
    half4_t pb;
    if constexpr (ONE) {
      const float pv = fast_exp2(__builtin_fmaf(lg.v[i], kLog2e, -msub));
      st.l += pv;
      pb = quad_gather_h4(pv * cb.sv[i] * vn, lr.psel);
    } else {
      float pv[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        pv[jj] = fast_exp2(__builtin_fmaf((float)lg.v[i][jj], kLog2e, -msub));
        st.l += pv[jj];
      }
      const float4_t svn = cb.sv[i] * vn;
      pb = (half4_t){(h16)(pv[0] * svn[0]), (h16)(pv[1] * svn[1]), (h16)(pv[2] * svn[2]), (h16)(pv[3] * svn[3])};
    }
    if constexpr (MORE) cb.sv[i] = load_scale<PRM, ONE>(p, vsrc.svp, i);
#pragma unroll
    for (int nt = 0; nt < CB::NT; ++nt) {
      const uint4 w4 = cb.vc[gr][nt];
      const uint32_t word = ii == 0 ? w4.x : ii == 1 ? w4.y : ii == 2 ? w4.z : w4.w;
      st.pacc[nt] = mfma_16x16x16(i8x4_to_h4(word), pb, st.pacc[nt]);
    }
    if constexpr (MORE) {
      if (ii == 3) {
        load_vc(p, vsrc, gr, cb);
        pin_vmem();
      }
    }
  }
}

// A sequence's tier counters, read once at the start of a workgroup into
// scalar registers: a counter read later, next to the prefetched codes,
// would make the compiler wait for every load in flight (vmcnt(0)).
struct SeqCounters {
  int ncold, tail_head, tail_len;
};
__device__ __forceinline__ SeqCounters read_counters(const DecodeParams& p, int b) {
  const int4 c = *reinterpret_cast<const int4*>(p.counters + b * SC_NCOUNTERS);  // NCOLD, TAIL_HEAD, TAIL_LEN, NEXT_POS
  SeqCounters s;
  s.ncold = __builtin_amdgcn_readfirstlane(c.x);
  s.tail_head = __builtin_amdgcn_readfirstlane(c.y);
  s.tail_len = __builtin_amdgcn_readfirstlane(c.z);
  return s;
}

// Softmax state carried through the tail tiles: running max (log2 domain),
// lane-partial sum and the accumulated rescale of the cold accumulators.
struct TailState {
  float m2, l, scale;
};

// Loads of one FP16 tail tile (16 tokens of one KV head): the key row of
// token t0 + n (RoPE pairs of lane group g), its position, and the quarter
// V row of token t0 + lane / 4 that the lane stages.
template <int D>
struct TailFetch {
  Half8s<Geo<D>::NV> kx1, kx2;
  half8_t vq[D / 32];
  int kpos;
  Half8s<Geo<D>::NV> c1, s1, c2, s2;  // RoPE entries at kpos (tail_fetch_rope); c2/s2 when the halves differ
};

// ok = false (no tail tile for this unit) still issues the loads, from the
// first D elements of Q and the sequence's counters, so that callers can
// prefetch without a branch: a branch around loads leaves the wait counts
// after it conservative, and later waits would also cover unrelated loads.
template <int D>
__device__ __forceinline__ void tail_fetch(const DecodeParams& p, int b, int h, int t0, int tl, int th, bool ok,
                                           TailFetch<D>& f) {
  using G = Geo<D>;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const long bh = (long)(b * p.Hkv + h);
  const int cap = p.TCAP > 0 ? p.TCAP : 1;
  const int t = t0 + n;
  const int slot = ok ? (th + (t < tl ? t : 0)) % cap : 0;
  const int32_t* pos = ok ? p.tail_pos + (long)b * p.TCAP : p.counters;
  const h16* kb = ok ? p.tail_k + bh * p.TCAP * D : p.q;
  const h16* vb = ok ? p.tail_v + bh * p.TCAP * D : p.q;
  f.kpos = pos[slot];
  const h16* krow = kb + (long)slot * D + g * G::QG;
  f.kx1 = load_h8s<G::NV>(krow);
  f.kx2 = load_h8s<G::NV>(krow + G::HALF);
  const int t2 = t0 + (lane >> 2);
  const int vslot = ok ? (th + (t2 < tl ? t2 : 0)) % cap : 0;
  const h16* vrow = vb + (long)vslot * D + (lane & 3) * (D / 4);
#pragma unroll
  for (int q = 0; q < D / 32; ++q) f.vq[q] = *reinterpret_cast<const half8_t*>(vrow + 8 * q);
}

// The RoPE table entries of the key a lane rotates (position f.kpos), issued
// once the position has arrived.
template <int D, bool HE>
__device__ __forceinline__ void tail_fetch_rope(const DecodeParams& p, bool rope, TailFetch<D>& f) {
  using G = Geo<D>;
  const int g = (threadIdx.x & 63) >> 4;
  if (rope) {
    const long r = (long)clamp_angle(f.kpos, p.rope_len) * p.rope_stride + g * G::QG;
    f.c1 = load_h8s<G::NV>(p.cos + r);
    f.s1 = load_h8s<G::NV>(p.sin + r);
    if constexpr (!HE) {
      f.c2 = load_h8s<G::NV>(p.cos + r + G::HALF);
      f.s2 = load_h8s<G::NV>(p.sin + r + G::HALF);
    }
  }
}

// One FP16 tail tile (tokens t0 .. t0 + 15 of one KV head, loads in f),
// merged into the wave's running softmax state.  Scores use the fp16
// pre-RoPE keys rotated at their stored positions; P.V accumulates in oacc
// (O^T layout: lane (g, n) holds O[query column n][16 mt + 4 g + jj]).  The
// V tile is transposed through a wave-private LDS region.
template <int D, bool GEN, bool HE>
__device__ __forceinline__ void tail_tile(const DecodeParams& p, int b, int h, int t0, int tl, int ncold,
                                          const half8_t (&qb)[Geo<D>::DS], h16* vs, TailFetch<D> f, TailState& sm,
                                          float4_t (&oacc)[Geo<D>::MT]) {
  using G = Geo<D>;
  constexpr bool ONE = !GEN;
  constexpr int QPR = D / 32;  // 16-byte chunks per quarter of a V row
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int vr = lane >> 2, vqtr = lane & 3;
  const Lanes lr = lane_roles<ONE>(n, p.nrep);
  const bool rope = !GEN || p.rope_mode != SC_ROPE_NONE;
  if (t0 + n >= tl) {
#pragma unroll
    for (int v = 0; v < G::NV; ++v) f.kx1.v[v] = f.kx2.v[v] = (half8_t)(h16)0;
  }
  if (t0 + vr >= tl) {
#pragma unroll
    for (int q = 0; q < QPR; ++q) f.vq[q] = (half8_t)(h16)0;
  }
  half8_t ya[G::DS];
  if (!rope) {
    unrotated<D>(f.kx1, f.kx2, ya);
  } else {
    if constexpr (HE) {
      rotate_he<D>(f.kx1, f.kx2, f.c1, f.s1, ya);
    } else {
      rotate<D>(f.kx1, f.kx2, f.c1, f.s1, f.c2, f.s2, p.rope_mode == SC_ROPE_DISTANCE ? kRotDist : kRotTailAbs,
                ya);
    }
  }
  // stage the V tile ([16 tokens][kVRow]); 8-byte stores, wave-private
#pragma unroll
  for (int q = 0; q < QPR; ++q) {
    h16* dst = vs + vr * kVRow + vqtr * (D / 4) + 8 * q;
    const half8_t v = f.vq[q];
    *reinterpret_cast<half4_t*>(dst) = (half4_t){v[0], v[1], v[2], v[3]};
    *reinterpret_cast<half4_t*>(dst + 4) = (half4_t){v[4], v[5], v[6], v[7]};
  }
  float4_t sacc = (float4_t)0.f;
#pragma unroll
  for (int s = 0; s < G::DS; ++s) sacc = mfma_16x16x32(ya[s], qb[s], sacc);
  half4_t pb;
  float alpha;
  if constexpr (ONE) {
    const bool valid = lr.valid && t0 + 4 * g + (n & 3) < tl;
    const float l16 = (float)fp16_logit(pick4(sacc, lr), p.scale);
    const float lg = valid ? l16 : -INFINITY;
    const float mt = head_max<ONE>(lg * kLog2e);
    const float m_new = fmaxf(sm.m2, mt);
    const float msub = (m_new == -INFINITY) ? 0.f : m_new;
    alpha = fast_exp2(sm.m2 - msub);
    sm.m2 = m_new;
    sm.l *= alpha;
    sm.scale *= alpha;  // rescale of the cold accumulators (applied by the caller)
    const float pv = fast_exp2(__builtin_fmaf(lg, kLog2e, -msub));
    sm.l += pv;
    pb = quad_gather_h4(pv, lr.psel);
  } else {
    const long cache_off = (long)ncold * p.TB;  // tail follows the cold blocks in cache order
    const bool hv = n < p.nrep;
    half4_t lg1[1];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int tk = t0 + 4 * g + jj;
      const bool valid = tk < tl;
      h16 l16 = fp16_logit(sacc[jj], p.scale);
      if constexpr (GEN) {
        if (p.logits && hv && valid)
          p.logits[b * p.lg_sb + (long)(h * p.nrep + n) * p.lg_sh + cache_off + tk] = (float)l16;
        if (p.mask && hv && valid && p.mask[b * p.mask_sb + (long)(h * p.nrep + n) * p.mask_sh + cache_off + tk] == 0)
          l16 = (h16)(-INFINITY);
      }
      lg1[0][jj] = valid ? l16 : (h16)(-INFINITY);
    }
    const float mt = head_max<ONE>(lane_max_log2<1>(lg1));
    const float m_new = fmaxf(sm.m2, mt);
    const float msub = (m_new == -INFINITY) ? 0.f : m_new;
    alpha = fast_exp2(sm.m2 - msub);
    sm.m2 = m_new;
    sm.l *= alpha;
    sm.scale *= alpha;
    float pv[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      pv[jj] = fast_exp2(__builtin_fmaf((float)lg1[0][jj], kLog2e, -msub));
      sm.l += pv[jj];
    }
    pb = (half4_t){(h16)pv[0], (h16)pv[1], (h16)pv[2], (h16)pv[3]};
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const h16* vt = vs + 4 * g * kVRow + n;
#pragma unroll
  for (int m = 0; m < G::MT; ++m) {
    const half4_t va = {vt[16 * m], vt[kVRow + 16 * m], vt[2 * kVRow + 16 * m], vt[3 * kVRow + 16 * m]};
    oacc[m] = mfma_16x16x16(va, pb, oacc[m] * alpha);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Tail tiles j, j + W, ... (W workgroups per sequence and head group) for a
// workgroup's wave; `first` holds the already issued loads of tile j.
template <int D, bool GEN, bool HE>
__device__ __forceinline__ void tail_tiles(const DecodeParams& p, const SeqCounters& sc, int b, int h, int j,
                                           const half8_t (&qb)[Geo<D>::DS], char* vstage, const TailFetch<D>& first,
                                           TailState& sm, float4_t (&oacc)[Geo<D>::MT]) {
  const int tl = sc.tail_len, th = sc.tail_head, ncold = sc.ncold;
  const int ntile = (tl + kTile - 1) / kTile;
  h16* vs = reinterpret_cast<h16*>(vstage);
  tail_tile<D, GEN, HE>(p, b, h, j * kTile, tl, ncold, qb, vs, first, sm, oacc);
  for (int tt = j + p.units_per_bh; tt < ntile; tt += p.units_per_bh) {
    TailFetch<D> f;
    tail_fetch<D>(p, b, h, tt * kTile, tl, th, true, f);
    tail_fetch_rope<D, HE>(p, !GEN || p.rope_mode != SC_ROPE_NONE, f);
    tail_tile<D, GEN, HE>(p, b, h, tt * kTile, tl, ncold, qb, vs, f, sm, oacc);
  }
}

// Writes a wave's partial record: lane (g, n) holds o[column n][16 mt + 4 g
// + jj]; query column n is head n (ONE = false) or head n >> 2 (ONE = true,
// written by quad lane 0).
template <int D, bool ONE>
__device__ __forceinline__ void write_record(const DecodeParams& p, int b, int h, int unit, const Lanes& lr,
                                             const float4_t (&o)[Geo<D>::MT], float m2, float l) {
  using G = Geo<D>;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const bool wr = lr.valid && (!ONE || (n & 3) == 0);
  const int hh = ONE ? n >> 2 : n;
  float* rec = record_ptr(p, b, h, unit, wr ? hh : 0, G::PREC);
#pragma unroll
  for (int mt = 0; mt < G::MT; ++mt)
    if (wr) *reinterpret_cast<float4_t*>(rec + 4 + 16 * mt + 4 * g) = o[mt];
  if (wr && g == 0) {
    rec[0] = m2;
    rec[1] = l;
  }
}

// Total of a lane-partial sum over the lanes of one query head.
template <bool ONE>
__device__ __forceinline__ float head_sum(float v) {
  v = sum_over_rows(v);
  return ONE ? quad_sum(v) : v;
}

// Unit j of (sequence b, group of four KV heads hq): wave w is KV head
// 4 hq + w.  Cold block j (if the sequence has it) is walked in ranges of
// T = 16 TPW tokens; the RoPE rows of a range are staged once per
// workgroup in LDS (double-buffered) and the INT8 codes of the next range
// are in flight (ping-pong register buffers) while the current one is
// processed.  Then tail tile j (16 FP16 tokens, if present) is folded in.
// Each wave writes one partial record per unit.
template <int D, int KK, int KV, int TPW, bool GEN, bool HE, int PRM>
__device__ void cold_unit(const DecodeParams& p, int b, int hq, int j, char* smem) {
  using G = Geo<D>;
  constexpr bool ONE = !GEN;
  using CB = CodeBuf<KK, KV, TPW, ONE>;
  using RS = RopeStage<D, HE>;
  constexpr int T = kTile * TPW;
  constexpr int NT = KV / 16;
  constexpr int KC = CB::KC;
  const int lane = threadIdx.x & 63, g = lane >> 4, n = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: per-head bases in SGPRs
  const int h = hq * kWaves + w;
  const bool young = (int)(blockIdx.x >> 3) >= p.young_slot;
  // The branch-free path runs only when the KV heads fill whole groups of
  // four: with no idle wave, its loads are issued without branches.
  const bool hvalid = !GEN || h < p.Hkv;
  const int nrep = p.nrep;
  const Lanes lr = lane_roles<ONE>(n, nrep);
  const int qhead = ONE ? n >> 2 : n;  // query head of this lane's MFMA column
  const SeqCounters sc = read_counters(p, b);
  const int ncold = sc.ncold;
  const int jb = j / p.split;                  // cold block of this unit
  const int nR = p.TB / T / p.split;           // ranges of this unit
  const int r0 = (j - jb * p.split) * nR;      // its first range within the block
  if (jb >= ncold) {  // uniform over the workgroup: no cold block, tail tiles only
    if (!hvalid) return;
    half8_t qt[G::DS];
    if (lr.valid) {
      load_q<D>(p, b, h, g, qhead, qt);
    } else {
#pragma unroll
      for (int s = 0; s < G::DS; ++s) qt[s] = (half8_t)(h16)0;
    }
    TailState sm;
    sm.m2 = -INFINITY;
    sm.l = 0.f;
    sm.scale = 0.f;
    float4_t oacc[G::MT];
#pragma unroll
    for (int m = 0; m < G::MT; ++m) oacc[m] = (float4_t)0.f;
    const bool he = !GEN || p.halves_equal != 0;
    if (p.fold_tail && j * kTile < sc.tail_len) {
      TailFetch<D> tf;
      tail_fetch<D>(p, b, h, j * kTile, sc.tail_len, sc.tail_head, true, tf);
      const bool trope = !GEN || p.rope_mode != SC_ROPE_NONE;
      if (he)
        tail_fetch_rope<D, true>(p, trope, tf);
      else
        tail_fetch_rope<D, false>(p, trope, tf);
      if (he)
        tail_tiles<D, GEN, true>(p, sc, b, h, j, qt, smem + w * kTile * kVRow * 2, tf, sm, oacc);
      else if constexpr (GEN)
        tail_tiles<D, GEN, false>(p, sc, b, h, j, qt, smem + w * kTile * kVRow * 2, tf, sm, oacc);
    }
    write_record<D, ONE>(p, b, h, j, lr, oacc, sm.m2, head_sum<ONE>(sm.l));
    return;
  }
  const long bhj = (long)(b * p.Hkv + (hvalid ? h : 0)) * p.NB + jb;
  const int start = p.block_start[b * p.NB + jb];
  const int qp = !p.qpos ? p.qpos_scalar : p.qpos64 ? (int)reinterpret_cast<const int64_t*>(p.qpos)[b] : p.qpos[b];
  const bool dist = p.rope_mode == SC_ROPE_DISTANCE;
  const bool rope = !GEN || p.rope_mode != SC_ROPE_NONE;
  constexpr int RBUF = T * RS::ROW;  // bytes of one staged range

  // ---- prologue: RoPE rows of range 0 (L2) first, then the HBM loads
  using SM = StageMap<D, HE, T>;
  const SM smap = stage_map<D, HE, T>(p, dist);
  U4s<2 * SM::NS> sv0{};  // range 0's RoPE rows: requested before the HBM loads, stored after them
  if (rope) sv0 = stage_fetch<D, HE, T>(p, smap, start + r0 * T, qp, dist);
  CB cb0;  // codes of the current range, refilled in place with the next
  half8_t a8[G::MT][KC];
  half4_t a4[G::MT];
  half8_t qb[G::DS];
  float vn = 1.f;
  if (hvalid) {
    load_codes<KK, PRM, ONE>(p, code_src<KK, KV>(p, bhj, r0 * T), cb0);
    // K basis as the A operand: row n of tile mt is d = perm(mt, n).
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
    if (lr.valid) {
      load_q<D>(p, b, h, g, qhead, qb);
    } else {
#pragma unroll
      for (int s = 0; s < G::DS; ++s) qb[s] = (half8_t)(h16)0;
    }
    vn = p.vnorm[bhj];
  }
  if (rope) stage_store<D, HE, T>(smem, smap, sv0);
  const long cache_tok = (long)jb * p.TB + r0 * T;  // cache-order index of the unit's first token
  const uint8_t* mrow = nullptr;
  float* lrow = nullptr;
  if constexpr (GEN) {
    mrow = (p.mask && lr.valid) ? p.mask + b * p.mask_sb + (long)(h * nrep + n) * p.mask_sh + cache_tok : nullptr;
    lrow = (p.logits && lr.valid) ? p.logits + b * p.lg_sb + (long)(h * nrep + n) * p.lg_sh + cache_tok : nullptr;
  }
  ColdState<KV> st;
  st.m2 = -INFINITY;
  st.l = 0.f;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) st.pacc[nt] = (float4_t)0.f;
  __syncthreads();

  // ---- ranges: step rr runs phase A of range rr, phase C of range rr - 1
  // (whose V codes are refilled with range rr's) and phase B of range rr.
  // The last range is peeled (no K refill, no staging) and its phase C
  // follows the loop.
  RangeLogits<ONE, TPW> lgp;  // logits of the previous range
  float msp = 0.f, alp = 1.f;
  auto step = [&](auto more_tag, auto prev_tag, int rr) __attribute__((always_inline)) {
    constexpr bool M = decltype(more_tag)::value;
    constexpr bool P = decltype(prev_tag)::value;
    char* cur = smem + (rr & 1) * RBUF;
    char* next = smem + ((rr + 1) & 1) * RBUF;
    if (hvalid) {
      RangeLogits<ONE, TPW> lg;
      range_scores<D, KK, KV, TPW, GEN, HE, PRM, M>(p, cb0, code_src<KK, KV>(p, bhj, (r0 + rr + 1) * T), a8, a4, qb,
                                                     smap, cur, next, start + (r0 + rr + 1) * T, qp, dist, rope,
                                                     mrow ? mrow + rr * T : nullptr, lrow ? lrow + rr * T : nullptr,
                                                     lg);
      if constexpr (P)
        range_values<KV, TPW, GEN, PRM, true>(p, cb0, code_src<KK, KV>(p, bhj, (r0 + rr) * T), lgp, msp, alp, vn, st);
      range_max<ONE, TPW>(lg, st, msp, alp);
      lgp = lg;
    } else if (M && rope) {
      // idle head slot: still stage its share of the next range's rows
      stage_store<D, HE, T>(next, smap, stage_fetch<D, HE, T>(p, smap, start + (r0 + rr + 1) * T, qp, dist));
    }
    __syncthreads();
    if (young && rr == kYoungPrioRange) __builtin_amdgcn_s_setprio(2);
  };
  using TT = std::integral_constant<bool, true>;
  using FF = std::integral_constant<bool, false>;
  if (nR > 2) {
    step(TT(), FF(), 0);
    for (int rr = 1; rr + 2 < nR; ++rr) step(TT(), TT(), rr);
  }
  // the FP16 tail tile of this workgroup is loaded during the last two
  // ranges and the V basis of the final projection during the last one (the
  // basis too would spill registers in the second-to-last)
  TailFetch<D> tf;
  const int tl = sc.tail_len;
  const bool has_tail = p.fold_tail && hvalid && j * kTile < tl;
  tail_fetch<D>(p, b, h, j * kTile, tl, sc.tail_head, has_tail, tf);
  half4_t bvf[G::MT][NT];
  const h16* bvb = p.basis_v + bhj * (long)D * KV;
  auto load_bv = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int mt = 0; mt < G::MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        bvf[mt][nt] = *reinterpret_cast<const half4_t*>(bvb + (long)(16 * mt + n) * KV + 16 * nt + 4 * g);
  };
  // With the smaller ranks of the branch-free path the tail tile's RoPE
  // entries (its positions arrived during the range before) are requested
  // before the last range, whose step stages no rows and refills no codes,
  // so they arrive while it computes; elsewhere the registers are not there
  // (k = 32/32: 36 spills) and they follow the last range.
  constexpr bool kEarlyTailRope = !GEN && KK + KV <= 48;
  if (nR > 2) {
    step(TT(), TT(), nR - 2);
    load_bv();
    if constexpr (kEarlyTailRope) tail_fetch_rope<D, HE>(p, rope, tf);
    step(FF(), TT(), nR - 1);
  } else if (nR == 2) {
    step(TT(), FF(), 0);
    load_bv();
    if constexpr (kEarlyTailRope) tail_fetch_rope<D, HE>(p, rope, tf);
    step(FF(), TT(), 1);
  } else {
    load_bv();
    if constexpr (kEarlyTailRope) tail_fetch_rope<D, HE>(p, rope, tf);
    step(FF(), FF(), 0);
  }
  if constexpr (!kEarlyTailRope)
    tail_fetch_rope<D, HE>(p, rope, tf);  // positions arrived during the last ranges (unconditional: no branch)
  if (hvalid) range_values<KV, TPW, GEN, PRM, false>(p, cb0, CodeSrc{}, lgp, msp, alp, vn, st);
  if (!hvalid) return;
  // ---- FP16 tail tiles of this workgroup, merged into the running state
  float4_t oacc[G::MT];
#pragma unroll
  for (int m = 0; m < G::MT; ++m) oacc[m] = (float4_t)0.f;
  if (has_tail) {
    TailState sm;
    sm.m2 = st.m2;
    sm.l = st.l;
    sm.scale = 1.f;  // collects the rescale of the cold accumulators
    tail_tiles<D, GEN, HE>(p, sc, b, h, j, qb, smem + w * kTile * kVRow * 2, tf, sm, oacc);
    st.m2 = sm.m2;
    st.l = sm.l;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) st.pacc[nt] *= sm.scale;
  }

  // ---- projection O^T[d][column] = B_V^T[d][i] . Pacc[i][column] on MFMA;
  // Pacc (coefficient i = 16 nt + 4 g + jj of column n, already the
  // B-operand layout) is split into fp16 hi + lo parts to keep fp32 accuracy.
  half4_t ph[NT], pl[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const h16 hi = (h16)st.pacc[nt][jj];
      ph[nt][jj] = hi;
      pl[nt][jj] = (h16)(st.pacc[nt][jj] - (float)hi);
    }
  const float ivn = 1.0f / vn;
  float4_t o[G::MT];
#pragma unroll
  for (int mt = 0; mt < G::MT; ++mt) {
    float4_t acc = (float4_t)0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      acc = mfma_16x16x16(bvf[mt][nt], ph[nt], acc);
      acc = mfma_16x16x16(bvf[mt][nt], pl[nt], acc);
    }
    o[mt] = acc * ivn + oacc[mt];
  }
  write_record<D, ONE>(p, b, h, j, lr, o, st.m2, head_sum<ONE>(st.l));
}

// Workgroup x runs on XCD x % 8 (round-robin dispatch).  Each XCD gets a
// contiguous, equal share of the units in chunk-major order, so
// concurrently running units of one XCD read the same cos/sin rows from
// its L2.  Within the share, slots s and s + half (the two workgroups a CU
// holds) take consecutive units, i.e. the same block for two head groups.
template <int D, int KK, int KV, int TPW, bool GEN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void decode_partial_kernel(DecodeParams p) {
  extern __shared__ __align__(16) char smem[];
  const long xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  const long c_lo = xcd * p.n_cold_units / 8, c_hi = (xcd + 1) * p.n_cold_units / 8;
  if (slot >= c_hi - c_lo) return;
  const long n = c_hi - c_lo, half = (n + 1) / 2;
  const long u = c_lo + (slot < half ? 2 * slot : 2 * (slot - half) + 1);
  const int nbq = p.B * p.n_hq;
  const int j = (int)(u / nbq), bq = (int)(u % nbq);
  if constexpr (GEN) {
    if (p.rope_mode != SC_ROPE_NONE && !p.halves_equal)
      cold_unit<D, KK, KV, TPW, GEN, false, 2>(p, bq / p.n_hq, bq % p.n_hq, j, smem);
    else
      cold_unit<D, KK, KV, TPW, GEN, true, 2>(p, bq / p.n_hq, bq % p.n_hq, j, smem);
  } else {
    if (p.per_row)
      cold_unit<D, KK, KV, TPW, GEN, true, 1>(p, bq / p.n_hq, bq % p.n_hq, j, smem);
    else
      cold_unit<D, KK, KV, TPW, GEN, true, 0>(p, bq / p.n_hq, bq % p.n_hq, j, smem);
  }
}

// Log-sum-exp merge of the partial records of one (sequence, query head):
// one single-wave workgroup per query head, lane l owns d = E l .. E l + E - 1.
// Records are merged U at a time with every load of a chunk in flight at
// once: lane k (and k + 32 when U = 32) loads the (m, l) header of record k,
// the chunk maximum and the weighted sum of l are register reductions, and
// the weight of record k reaches every lane by readlane (an SGPR operand of
// the FMAs).  U = 64 when there are more than 32 records: each dependent
// round of loads then covers twice the records.
// Every unit writes its record (m = -inf, l = 0, o = 0 when it saw no
// token), so a weight of zero needs no branch.
// Reduction over each 32-lane half of a wavefront in registers: DPP quad
// permutes (lane ^ 1, lane ^ 2), row half-mirror and row mirror (every
// 16-lane row), then v_permlane16_swap between the two rows of the half.
template <bool MAX>
__device__ __forceinline__ float half_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
  v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  const uint32_t u = __float_as_uint(v);
  auto b = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return op(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Reduction of the chunk's headers: each 16-lane row (U = 16: every row holds
// the same headers), each 32-lane half (U = 32: both halves hold them), or
// the whole wave (U = 64).
template <bool MAX, int U>
__device__ __forceinline__ float chunk_reduce(float v) {
  static_assert(U == 16 || U == 32 || U == 64, "one header per lane of a row, a half or the wave");
  if constexpr (U == 16) {
    auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    return op(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)));
  }
  v = half_reduce<MAX>(v);
  if constexpr (U == 64) {
    const uint32_t u = __float_as_uint(v);
    auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    v = MAX ? fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1])) : __uint_as_float(a[0]) + __uint_as_float(a[1]);
  }
  return v;
}

// NW > 1: wave w merges the chunks starting at w U, w U + NW U, ..., so
// each wave's loads are one round; the waves' states are then merged by
// wave 0 through LDS after one barrier.
template <int D, int U, int NW>
__global__ __launch_bounds__(64 * NW) void decode_combine_kernel(DecodeParams p) {
  constexpr int PREC = Geo<D>::PREC;
  constexpr int E = D / 64;  // d values per lane
  const int wq = blockIdx.x;
  const int b = wq / p.Hq, qh = wq % p.Hq;
  const int h = qh / p.nrep, hh = qh % p.nrep;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int W = p.units_per_bh;
  const float* r0 = record_ptr(p, b, h, 0, hh, PREC);
  const long us = (long)p.nrep * PREC;
  float M = -INFINITY, L = 0.f, O[E];
#pragma unroll
  for (int e = 0; e < E; ++e) O[e] = 0.f;
  for (int u0 = wv * U; u0 < W; u0 += NW * U) {
    const int ku = u0 + (lane & (U - 1));
    const bool has = ku < W;
    const float* rh = r0 + (long)(has ? ku : u0) * us;
    const float2 ml = *reinterpret_cast<const float2*>(rh);
    float orr[U][E];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const float* r = r0 + (long)min(u0 + k, W - 1) * us + 4 + E * lane;
      if constexpr (E == 2) {
        const float2 v = *reinterpret_cast<const float2*>(r);
        orr[k][0] = v.x;
        orr[k][1] = v.y;
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) orr[k][e] = r[e];
      }
    }
    // Keep every load of the chunk above the reductions: left alone, the
    // scheduler sinks them to their uses and the chunk costs two round trips.
    __builtin_amdgcn_sched_barrier(0);
    const float mk = has ? ml.x : -INFINITY;
    const float mc = chunk_reduce<true, U>(mk);
    const float mn = fmaxf(M, mc);
    if (mn == -INFINITY) continue;  // wave-uniform: nothing seen yet
    const float ck = mk == -INFINITY ? 0.f : fast_exp2(mk - mn);
    const float lc = chunk_reduce<false, U>(has ? ml.y * ck : 0.f);
    const float a = fast_exp2(M - mn);  // exp2(-inf) = 0 on the first chunk
    L = L * a + lc;
#pragma unroll
    for (int e = 0; e < E; ++e) O[e] *= a;
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ck), k));
#pragma unroll
      for (int e = 0; e < E; ++e) O[e] = __builtin_fmaf(orr[k][e], c, O[e]);
    }
    M = mn;
  }
  if constexpr (NW > 1) {
    __shared__ float st[NW][2 + E * 64];  // per wave: M, L (wave-uniform), then O[e][lane]
    if (lane == 0) {
      st[wv][0] = M;
      st[wv][1] = L;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) st[wv][2 + e * 64 + lane] = O[e];
    __syncthreads();
    if (wv != 0) return;
    float mt = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) mt = fmaxf(mt, st[v][0]);
    L = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) O[e] = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float mv = st[v][0];
      const float a = mv == -INFINITY ? 0.f : fast_exp2(mv - mt);  // a wave that saw no token adds nothing
      L = __builtin_fmaf(st[v][1], a, L);
#pragma unroll
      for (int e = 0; e < E; ++e) O[e] = __builtin_fmaf(st[v][2 + e * 64 + lane], a, O[e]);
    }
  }
  h16* o = p.out + b * p.out_sb + (long)qh * p.out_sh + E * lane;
#pragma unroll
  for (int e = 0; e < E; ++e) o[e] = (h16)(O[e] / L);
}

bool padded_rank_ok(int kp) { return kp == 16 || kp == 32 || kp == 64; }

// Tiles of 16 tokens per wave and range (64-token ranges).
constexpr int kTilesPerWave = 4;

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
  if (a->grid_blocks > 0 && (((uintptr_t)t->codes_k & 15) || ((uintptr_t)t->codes_v & 15) ||
                             ((uintptr_t)t->basis_k & 15) || ((uintptr_t)t->basis_v & 15) ||
                             ((uintptr_t)t->scales_k & 3) || ((uintptr_t)t->scales_v & 3)))
    return sc_fail(SC_ERR_INVALID, "cold-tier arrays must be 16-byte aligned");
  if (a->grid_tail > 0 && (((uintptr_t)t->tail_k & 15) || ((uintptr_t)t->tail_v & 15)))
    return sc_fail(SC_ERR_INVALID, "tail arrays must be 16-byte aligned");
  const int tpw = kTilesPerWave;
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
  p->tpw = tpw;
  p->n_hq = (t->kv_heads + kWaves - 1) / kWaves;
  // The FP16 tail is processed by the cold workgroups: tail tile t (16
  // tokens) goes to workgroup t mod W of its sequence and head group, with
  // W = max(grid_blocks, tail tiles): workgroups past the cold blocks only
  // do tail work, and no workgroup gets more than one tail tile.
  const int tail_tiles_grid = (a->grid_tail + kTile - 1) / kTile;
  p->fold_tail = a->grid_tail > 0;
  // A cold block is split over `split` workgroups (consecutive 64-token
  // ranges each) while the doubled grid still holds at most kFillUnits
  // workgroups: small batches would otherwise leave most CUs idle while a
  // few workgroups walk whole blocks, and beyond one workgroup per CU the
  // extra workgroups' fixed cost (bases, tail tile, record, a longer merge)
  // outweighs the shorter walk (same-process sweeps over batch 1-4 and 4K-33K
  // contexts: this bound picked the fastest split in every case).
  const int ranges = t->block_size / (kTile * tpw);
  const long base_units = (long)a->grid_blocks * t->batch * ((t->kv_heads + kWaves - 1) / kWaves);
  if (a->split < 0 || ranges % (a->split > 0 ? a->split : 1) || (a->split & (a->split - 1)))
    return sc_fail(SC_ERR_INVALID, "split %d must be a power of two dividing block_size/64 = %d", a->split, ranges);
  p->split = a->split > 0 ? a->split : 1;
  if (a->split == 0)
    while (ranges % (2 * p->split) == 0 && base_units * p->split * 2 <= kFillUnits) p->split *= 2;
  const int split_units = p->grid_blocks * p->split;
  p->cold_units = split_units > tail_tiles_grid ? split_units : tail_tiles_grid;
  p->units_per_bh = p->cold_units;
  p->n_cold_units = (long)p->cold_units * p->B * p->n_hq;
  p->scale = a->scale;
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
  p->qpos64 = a->query_pos_i64 != 0;
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

// Compute units per XCD of the current device (8 XCDs), cached per device.
int cus_per_xcd() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 32;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 8) n = 256;
    v = n / 8;
    cache[dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

size_t workspace_bytes(const DecodeParams& p, int D) {
  return (size_t)p.B * p.Hkv * p.units_per_bh * p.nrep * (D + 4) * sizeof(float);
}

template <int D, int KK, int KV, int TPW, bool GEN>
int launch(DecodeParams& p, hipStream_t s) {
  long slots = 0;
  for (int x = 0; x < 8; ++x) {
    const long nc = (x + 1) * p.n_cold_units / 8 - x * p.n_cold_units / 8;
    if (nc > slots) slots = nc;
  }
  const long grid = 8 * slots;
  size_t lds = 0;
  if (p.cold_units > 0 && (GEN ? p.rope_mode != SC_ROPE_NONE : true)) {
    const bool he = !GEN || p.halves_equal;
    lds = (size_t)2 * kTile * TPW * (he ? RopeStage<D, true>::ROW : RopeStage<D, false>::ROW);
  }
  if (p.fold_tail) {
    const size_t stage_fold = (size_t)kWaves * kTile * kVRow * 2;  // one V tile per wave
    if (stage_fold > lds) lds = stage_fold;
  }
  if (grid > 0) {
    hipLaunchKernelGGL((decode_partial_kernel<D, KK, KV, TPW, GEN>), dim3((unsigned)grid), dim3(kThreads), lds, s, p);
    int rc = sc_launch_status("decode_partial_kernel");
    if (rc) return rc;
  }
  // Records per round (U) and waves (NW) so that one round covers the
  // records where it can: same-process timings preferred two waves with
  // smaller rounds over one wave with larger ones (batch 1 x 4K, 56 records:
  // 10.89 -> 10.41 us per call), and were equal at 32 records.
  const int W = p.units_per_bh;
  if (W > 128)
    hipLaunchKernelGGL((decode_combine_kernel<D, 64, 4>), dim3(p.B * p.Hq), dim3(256), 0, s, p);
  else if (W > 64)
    hipLaunchKernelGGL((decode_combine_kernel<D, 32, 4>), dim3(p.B * p.Hq), dim3(256), 0, s, p);
  else if (W > 32)
    hipLaunchKernelGGL((decode_combine_kernel<D, 32, 2>), dim3(p.B * p.Hq), dim3(128), 0, s, p);
  else if (W > 16)
    hipLaunchKernelGGL((decode_combine_kernel<D, 16, 2>), dim3(p.B * p.Hq), dim3(128), 0, s, p);
  else
    hipLaunchKernelGGL((decode_combine_kernel<D, 16, 1>), dim3(p.B * p.Hq), dim3(64), 0, s, p);
  return sc_launch_status("decode_combine_kernel");
}

template <int D, int KK, int KV, bool GEN>
int dispatch_tpw(DecodeParams& p, hipStream_t s) {
  return launch<D, KK, KV, kTilesPerWave, GEN>(p, s);
}

template <int D, int KK, bool GEN>
int dispatch_kv(DecodeParams& p, int kv, hipStream_t s) {
  switch (kv) {
    case 16: return dispatch_tpw<D, KK, 16, GEN>(p, s);
    case 32: return dispatch_tpw<D, KK, 32, GEN>(p, s);
    default: return dispatch_tpw<D, KK, 64, GEN>(p, s);
  }
}

template <int D, bool GEN>
int dispatch_kk(DecodeParams& p, int kk, int kv, hipStream_t s) {
  switch (kk) {
    case 16: return dispatch_kv<D, 16, GEN>(p, kv, s);
    case 32: return dispatch_kv<D, 32, GEN>(p, kv, s);
    default: return dispatch_kv<D, 64, GEN>(p, kv, s);
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

namespace {

// Launches the partial and combine kernels with the records at ws (of at
// least workspace_bytes(p) bytes, checked by the caller).
int decode_launch(const ScDecodeArgs* args, DecodeParams& p, float* ws, void* stream) {
  const int D = args->tier->head_dim;
  p.ws = ws;
  p.young_slot = cus_per_xcd();
  hipStream_t s = (hipStream_t)stream;
  const int kk = args->tier->kp_keys, kv = args->tier->kp_values;
  // The branch-free path keeps one logit per lane, which needs GQA groups
  // of at most 4 query heads, and has no idle waves (KV heads a multiple of 4).
  const bool gen = args->mask || args->logits_out || args->rope_mode == SC_ROPE_NONE || !args->halves_equal ||
                   args->q_heads / args->tier->kv_heads > 4 || args->tier->kv_heads % kWaves != 0;
  if (D == 128)
    return gen ? dispatch_kk<128, true>(p, kk, kv, s) : dispatch_kk<128, false>(p, kk, kv, s);
  return gen ? dispatch_kk<64, true>(p, kk, kv, s) : dispatch_kk<64, false>(p, kk, kv, s);
}

}  // namespace

extern "C" int sc_decode_attn(const ScDecodeArgs* args, void* workspace, size_t workspace_bytes_, void* stream) {
  DecodeParams p;
  int rc = fill_params(args, &p);
  if (rc) return rc;
  const size_t need = workspace_bytes(p, args->tier->head_dim);
  if (!workspace || workspace_bytes_ < need)
    return sc_fail(SC_ERR_WORKSPACE, "decode workspace too small: %zu < %zu bytes", workspace_bytes_, need);
  if (p.units_per_bh == 0) return sc_fail(SC_ERR_INVALID, "empty cache: no blocks and no tail scanned");
  return decode_launch(args, p, (float*)workspace, stream);
}
