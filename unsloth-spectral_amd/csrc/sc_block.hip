// Per-block score and value products of the reference's kernels module
// (gfx950): the API helpers that work on one block's dequantised
// coefficients, outside the fused decode kernel.
//
// scores  -- spectral_score_forward, kernels/spectral_attention.py:375-453:
//            Q aligned by the inverse RoPE at each key's absolute position
//            (fp16 elementwise, _apply_inverse_rope :340-372), projected on
//            the basis in fp32, times the coefficients, summed in fp32 and
//            rounded to fp16.
// values  -- spectral_value_forward, kernels/spectral_attention.py:544-601:
//            v_lat = P . C_V in fp32, out = v_lat . B_V in fp32, rounded to
//            fp16.
// GQA: query head h reads KV head h / (q_heads / kv_heads) (repeat_interleave).
#include "sc_common.h"

namespace {

struct BlockParams {
  int B, Hq, Hkv, nrep, T, k, D;
  const h16* coeffs;  // [Hkv][T][k]
  const h16* basis;   // [Hkv][k][D]
};

// One wave per (sequence, query head, 64 tokens); lane = token.  The basis
// of the KV head and the query row are staged in LDS and read by every lane
// at the same address (broadcast).
constexpr int kScoreTokens = 64;

template <int D>
__global__ __launch_bounds__(kScoreTokens) void block_scores_kernel(BlockParams p, const h16* q, long q_sb,
                                                                    long q_sh, const h16* cos, const h16* sin,
                                                                    long rope_stride, int rope_len, int start,
                                                                    h16* out) {
  constexpr int HALF = D / 2;
  __shared__ __align__(16) h16 sb[64 * D];
  __shared__ __align__(16) h16 sq[D];
  const int t0 = blockIdx.x * kScoreTokens, hq = blockIdx.y, b = blockIdx.z;
  const int h = hq / p.nrep, lane = threadIdx.x;
  const h16* bas = p.basis + (long)h * p.k * D;
  for (int i = lane; i < p.k * D / 8; i += kScoreTokens)
    reinterpret_cast<uint4*>(sb)[i] = reinterpret_cast<const uint4*>(bas)[i];
  const h16* qrow = q + b * q_sb + (long)hq * q_sh;
  for (int i = lane; i < D / 8; i += kScoreTokens)
    reinterpret_cast<uint4*>(sq)[i] = reinterpret_cast<const uint4*>(qrow)[i];
  __syncthreads();
  const int t = t0 + lane;
  if (t >= p.T) return;
  const int pos = min(max(start + t, 0), rope_len - 1);
  const h16* cr = cos + (long)pos * rope_stride;
  const h16* sr = sin + (long)pos * rope_stride;
  // inverse RoPE: (x1 c1 - x2 (-s1), x2 c2 + x1 (-s2)) in fp16, each product
  // and each sum rounded to fp16 as torch's elementwise fp16 ops round
  // (the products are kept apart from the sums: no fused multiply-add)
  float qa[D];
#pragma unroll
  for (int i = 0; i < HALF; ++i) {
    const h16 x1 = sq[i], x2 = sq[HALF + i];
    const h16 c1 = cr[i], c2 = cr[HALF + i];
    const h16 s1 = -sr[i], s2 = -sr[HALF + i];
    qa[i] = (float)(h16)(rounded<h16>(x1 * c1) - rounded<h16>(x2 * s1));
    qa[HALF + i] = (float)(h16)(rounded<h16>(x2 * c2) + rounded<h16>(x1 * s2));
  }
  const h16* crow = p.coeffs + ((long)h * p.T + t) * p.k;
  float acc = 0.f;
  for (int kk = 0; kk < p.k; ++kk) {
    const h16* brow = sb + kk * D;
    float lat = 0.f;
#pragma unroll
    for (int d = 0; d < D; d += 8) {
      const half8_t v = *reinterpret_cast<const half8_t*>(brow + d);
#pragma unroll
      for (int j = 0; j < 8; ++j) lat = __builtin_fmaf(qa[d + j], (float)v[j], lat);
    }
    acc = __builtin_fmaf(lat, (float)crow[kk], acc);
  }
  out[((long)b * p.Hq + hq) * p.T + t] = (h16)acc;
}

// One workgroup per (sequence, query head).  Thread (g, kk) sums the
// probabilities times coefficient kk over tokens g, g + G, ...; the G partial
// sums of each kk are added in LDS in a fixed order; then thread d forms
// out[d] = sum_kk v_lat[kk] * B_V[kk][d].
constexpr int kValueThreads = 256;

__global__ __launch_bounds__(kValueThreads) void block_values_kernel(BlockParams p, const float* attn, long a_sb,
                                                                     long a_sh, h16* out) {
  __shared__ float part[kValueThreads];
  __shared__ float vlat[64];
  const int hq = blockIdx.x, b = blockIdx.y, h = hq / p.nrep;
  const int tid = threadIdx.x;
  const int G = kValueThreads / p.k;  // token groups; threads from G * k on only write zeros
  const int g = tid / p.k, kk = tid % p.k;
  const float* arow = attn + b * a_sb + (long)hq * a_sh;
  const h16* cbase = p.coeffs + (long)h * p.T * p.k;
  float s = 0.f;
  if (g < G)
    for (int t = g; t < p.T; t += G) s = __builtin_fmaf(arow[t], (float)cbase[(long)t * p.k + kk], s);
  part[tid] = s;
  __syncthreads();
  if (tid < p.k) {
    float v = 0.f;
    for (int i = 0; i < G; ++i) v += part[i * p.k + tid];
    vlat[tid] = v;
  }
  __syncthreads();
  const h16* bas = p.basis + (long)h * p.k * p.D;
  for (int d = tid; d < p.D; d += kValueThreads) {
    float o = 0.f;
    for (int i = 0; i < p.k; ++i) o = __builtin_fmaf(vlat[i], (float)bas[(long)i * p.D + d], o);
    out[((long)b * p.Hq + hq) * p.D + d] = (h16)o;
  }
}

int check_block(int batch, int q_heads, int kv_heads, int tokens, int rank, int head_dim, const void* coeffs,
                const void* basis, BlockParams* p) {
  if (batch < 1 || kv_heads < 1 || q_heads < kv_heads || q_heads % kv_heads)
    return sc_fail(SC_ERR_INVALID, "q_heads %d must be a positive multiple of kv_heads %d", q_heads, kv_heads);
  if (tokens < 1) return sc_fail(SC_ERR_INVALID, "block of %d tokens", tokens);
  if (rank < 1 || rank > 64) return sc_fail(SC_ERR_UNSUPPORTED, "rank %d outside [1, 64]", rank);
  if (head_dim != 64 && head_dim != 128) return sc_fail(SC_ERR_UNSUPPORTED, "head_dim %d (64 or 128)", head_dim);
  if (!coeffs || !basis) return sc_fail(SC_ERR_INVALID, "null coefficients or basis");
  if (((uintptr_t)basis & 15)) return sc_fail(SC_ERR_INVALID, "basis must be 16-byte aligned");
  p->B = batch;
  p->Hq = q_heads;
  p->Hkv = kv_heads;
  p->nrep = q_heads / kv_heads;
  p->T = tokens;
  p->k = rank;
  p->D = head_dim;
  p->coeffs = (const h16*)coeffs;
  p->basis = (const h16*)basis;
  return SC_OK;
}

}  // namespace

extern "C" int sc_block_scores(const void* q, int64_t q_stride_b, int64_t q_stride_h, int32_t batch,
                               int32_t q_heads, const void* coeffs_k, const void* basis_k, int32_t kv_heads,
                               int32_t tokens, int32_t rank, int32_t head_dim, const void* cos, const void* sin,
                               int64_t rope_stride, int32_t rope_len, int32_t start_position, void* scores,
                               void* stream) {
  BlockParams p;
  int rc = check_block(batch, q_heads, kv_heads, tokens, rank, head_dim, coeffs_k, basis_k, &p);
  if (rc) return rc;
  if (!q || !scores || !cos || !sin || rope_len < 1 || rope_stride < head_dim)
    return sc_fail(SC_ERR_INVALID, "sc_block_scores: null or malformed q / scores / RoPE tables");
  if (((uintptr_t)q & 15) || (q_stride_b & 7) || (q_stride_h & 7))
    return sc_fail(SC_ERR_INVALID, "q rows must be 16-byte aligned");
  if (start_position < 0 || (int64_t)start_position + tokens > rope_len)
    return sc_fail(SC_ERR_INVALID, "key positions [%d, %d) outside the RoPE tables (%d rows)", start_position,
                   start_position + tokens, rope_len);
  const dim3 grid((tokens + kScoreTokens - 1) / kScoreTokens, q_heads, batch);
  hipStream_t s = (hipStream_t)stream;
  if (head_dim == 128)
    hipLaunchKernelGGL(block_scores_kernel<128>, grid, dim3(kScoreTokens), 0, s, p, (const h16*)q, (long)q_stride_b,
                       (long)q_stride_h, (const h16*)cos, (const h16*)sin, (long)rope_stride, rope_len,
                       start_position, (h16*)scores);
  else
    hipLaunchKernelGGL(block_scores_kernel<64>, grid, dim3(kScoreTokens), 0, s, p, (const h16*)q, (long)q_stride_b,
                       (long)q_stride_h, (const h16*)cos, (const h16*)sin, (long)rope_stride, rope_len,
                       start_position, (h16*)scores);
  return sc_launch_status("block_scores_kernel");
}

extern "C" int sc_block_values(const float* attn, int64_t attn_stride_b, int64_t attn_stride_h, int32_t batch,
                               int32_t q_heads, const void* coeffs_v, const void* basis_v, int32_t kv_heads,
                               int32_t tokens, int32_t rank, int32_t head_dim, void* out, void* stream) {
  BlockParams p;
  int rc = check_block(batch, q_heads, kv_heads, tokens, rank, head_dim, coeffs_v, basis_v, &p);
  if (rc) return rc;
  if (!attn || !out) return sc_fail(SC_ERR_INVALID, "sc_block_values: null attn or out");
  hipLaunchKernelGGL(block_values_kernel, dim3(q_heads, batch), dim3(kValueThreads), 0, (hipStream_t)stream, p,
                     attn, (long)attn_stride_b, (long)attn_stride_h, (h16*)out);
  return sc_launch_status("block_values_kernel");
}
