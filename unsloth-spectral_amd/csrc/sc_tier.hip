// Tier manager kernels (gfx950): tail append and cold-block dequantisation.
//
// append   -- spectral_cache.py:164-232 (new-generation reset :176-189,
//             auto-increment positions :199-208, concat :215-229, counters
//             :231-232).  The FP16 tail is a ring of tail_capacity slots per
//             sequence; appending writes rows in place instead of torch.cat.
// dequant  -- get_kv, spectral_cache.py:557-612: fp16(code*scale) . basis.
#include "sc_common.h"

namespace {

constexpr int kThreads = 256;

struct AppendParams {
  ScTierDesc t;
  const h16* k_new;
  const h16* v_new;
  long sb, sh, st;
  const void* positions;  // int32, or int64 with SC_APPEND_POS_I64
  int t_new;
  int flags;
};

// Position i of the append's [batch][t_new] positions.
__device__ __forceinline__ int append_pos(const AppendParams& p, long i) {
  return (p.flags & SC_APPEND_POS_I64) ? (int)static_cast<const int64_t*>(p.positions)[i]
                                       : static_cast<const int32_t*>(p.positions)[i];
}

// New generation: the caller says so (SC_APPEND_RESET), or, with
// SC_APPEND_DETECT_RESET, the sequence's first new position lies below the
// next expected one (spectral_cache.py:176-189, compared per sequence here).
__device__ __forceinline__ bool append_resets(const AppendParams& p, const int32_t* cnt, int b) {
  if (p.flags & SC_APPEND_RESET) return true;
  return (p.flags & SC_APPEND_DETECT_RESET) && p.positions && cnt[SC_CNT_TOTAL] > 0 &&
         append_pos(p, (long)b * p.t_new) < cnt[SC_CNT_NEXT_POS];
}

// The rows fit the ring: tail length after the append <= capacity.
__device__ __forceinline__ bool append_fits(const AppendParams& p, const int32_t* cnt, bool reset) {
  return (reset ? 0 : cnt[SC_CNT_TAIL_LEN]) + p.t_new <= p.t.tail_capacity;
}

// Work item `rem` of sequence b = one 16-byte chunk of one K or V row.
__device__ __forceinline__ void append_item(const AppendParams& p, int b, long rem) {
  const int D = p.t.head_dim, cpr = D / 8;
  const int kind = (int)(rem % 2);
  rem /= 2;
  const int chunk = (int)(rem % cpr);
  rem /= cpr;
  const int tt = (int)(rem % p.t_new);
  const int h = (int)(rem / p.t_new);
  const int32_t* cnt = p.t.counters + b * SC_NCOUNTERS;
  const bool reset = append_resets(p, cnt, b);
  if (!append_fits(p, cnt, reset)) return;  // nothing written; the counter update records the status
  const int base_len = reset ? 0 : cnt[SC_CNT_TAIL_LEN];
  const int base_head = reset ? 0 : cnt[SC_CNT_TAIL_HEAD];
  const int slot = (base_head + base_len + tt) % p.t.tail_capacity;
  const h16* src = (kind ? p.v_new : p.k_new) + b * p.sb + h * p.sh + (long)tt * p.st + chunk * 8;
  h16* dst = (h16*)(kind ? p.t.tail_v : p.t.tail_k) +
             (((long)b * p.t.kv_heads + h) * p.t.tail_capacity + slot) * D + chunk * 8;
  *reinterpret_cast<half8_t*>(dst) = *reinterpret_cast<const half8_t*>(src);
  if (h == 0 && chunk == 0 && kind == 0) {
    const int pos = p.positions ? append_pos(p, (long)b * p.t_new + tt) : (reset ? 0 : cnt[SC_CNT_NEXT_POS]) + tt;
    p.t.tail_pos[(long)b * p.t.tail_capacity + slot] = pos;
  }
}

__global__ __launch_bounds__(kThreads) void append_copy_kernel(AppendParams p) {
  const long per_b = (long)p.t.kv_heads * p.t_new * (p.t.head_dim / 8) * 2;
  const long idx = (long)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= per_b * p.t.batch) return;
  append_item(p, (int)(idx / per_b), idx % per_b);
}

// Counter update of sequence b after its rows are written.
__device__ __forceinline__ void append_counters(const AppendParams& p, int b) {
  int32_t* cnt = p.t.counters + b * SC_NCOUNTERS;
  const bool reset = append_resets(p, cnt, b);
  if (!append_fits(p, cnt, reset)) {  // ring overflow: counters unchanged, status set
    cnt[SC_CNT_STATUS] = SC_ERR_CAPACITY;
    return;
  }
  if (reset) {
    for (int i = 0; i < SC_NCOUNTERS; ++i) cnt[i] = 0;
  }
  cnt[SC_CNT_TAIL_LEN] += p.t_new;
  cnt[SC_CNT_NEXT_POS] += p.t_new;
  cnt[SC_CNT_TOTAL] += p.t_new;
}

__global__ void append_finalize_kernel(AppendParams p) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= p.t.batch) return;
  append_counters(p, b);
}

// Short appends (a decode step's token): one workgroup per sequence writes
// the sequence's rows, then, after a barrier, its counters.  Every thread
// reads the counters before the barrier and only thread 0 writes them after
// it, so the rows and the counter update need no second launch.
__global__ __launch_bounds__(kThreads) void append_short_kernel(AppendParams p) {
  const int b = blockIdx.x;
  const int D = p.t.head_dim, cpr = D / 8;
  const int per_b = p.t.kv_heads * p.t_new * cpr * 2;
  for (int i = threadIdx.x; i < per_b; i += kThreads) append_item(p, b, i);
  __syncthreads();
  if (threadIdx.x == 0) append_counters(p, b);
}

struct DequantParams {
  ScTierDesc t;
  int first, count;
  h16* k_out;
  h16* v_out;
};

// One thread per output element (b, h, token, d) of K and of V.  The
// coefficient is rounded twice, as the reference stores it: code * scale to
// fp32, then to fp16 (spectral_cache.py:404).
__global__ __launch_bounds__(kThreads) void dequant_kernel(DequantParams p) {
  const ScTierDesc& T = p.t;
  const int D = T.head_dim, TB = T.block_size;
  const long ntok = (long)p.count * TB;
  const long per_bh = ntok * D;
  const long idx = (long)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= per_bh * T.batch * T.kv_heads) return;
  const long bh = idx / per_bh;
  const long rem = idx % per_bh;
  const int tok = (int)(rem / D), d = (int)(rem % D);
  const int blk = p.first + tok / TB, t = tok % TB;
  const long bhj = bh * T.max_blocks + blk;
  const bool per_row = T.granularity == SC_QUANT_PER_ROW;
  const float sk = T.scales_k[per_row ? bhj * TB + t : bhj];
  const float sv = T.scales_v[per_row ? bhj * TB + t : bhj];
  const int8_t* ck = T.codes_k + bhj * TB * T.kp_keys + (long)t * T.kp_keys;
  const int8_t* cv = T.codes_v + bhj * T.kp_values * TB + t;
  const h16* bk = (const h16*)T.basis_k + bhj * (long)D * T.kp_keys + (long)d * T.kp_keys;
  const h16* bv = (const h16*)T.basis_v + bhj * (long)D * T.kp_values + (long)d * T.kp_values;
  float ak = 0.f, av = 0.f;
  for (int i = 0; i < T.k_keys; ++i) ak += (float)(h16)rounded((float)ck[i] * sk) * (float)bk[i];
  for (int i = 0; i < T.k_values; ++i) av += (float)(h16)rounded((float)cv[(long)i * TB] * sv) * (float)bv[i];
  p.k_out[idx] = (h16)ak;
  p.v_out[idx] = (h16)av;
}

}  // namespace

extern "C" int sc_tier_append(const ScTierDesc* t, const void* k_new, const void* v_new, int64_t stride_b,
                              int64_t stride_h, int64_t stride_t, const int32_t* positions, int32_t t_new,
                              int32_t flags, void* stream) {
  if (!t || !t->counters || !t->tail_k || !t->tail_v || !t->tail_pos)
    return sc_fail(SC_ERR_INVALID, "sc_tier_append: null tier");
  if (t_new < 0) return sc_fail(SC_ERR_INVALID, "negative t_new");
  if (flags & ~(SC_APPEND_DETECT_RESET | SC_APPEND_RESET | SC_APPEND_POS_I64))
    return sc_fail(SC_ERR_INVALID, "bad append flags %d", flags);
  if (t_new == 0) return SC_OK;
  if (t_new > t->tail_capacity)
    return sc_fail(SC_ERR_CAPACITY, "append of %d tokens exceeds the tail ring (%d)", t_new, t->tail_capacity);
  if (t->head_dim % 8) return sc_fail(SC_ERR_UNSUPPORTED, "head_dim must be a multiple of 8");
  if (!k_new || !v_new) return sc_fail(SC_ERR_INVALID, "null k_new/v_new");
  if (((uintptr_t)k_new & 15) || ((uintptr_t)v_new & 15) || (stride_b & 7) || (stride_h & 7) || (stride_t & 7))
    return sc_fail(SC_ERR_INVALID, "k_new/v_new rows must be 16-byte aligned");
  AppendParams p;
  p.t = *t;
  p.k_new = (const h16*)k_new;
  p.v_new = (const h16*)v_new;
  p.sb = stride_b;
  p.sh = stride_h;
  p.st = stride_t;
  p.positions = positions;
  p.t_new = t_new;
  p.flags = flags;
  const long per_b = (long)t->kv_heads * t_new * (t->head_dim / 8) * 2;
  const long items = (long)t->batch * per_b;
  hipStream_t s = (hipStream_t)stream;
  if (per_b <= 4 * kThreads) {  // one workgroup per sequence, counters in the same launch
    hipLaunchKernelGGL(append_short_kernel, dim3((unsigned)t->batch), dim3(kThreads), 0, s, p);
    return sc_launch_status("append_short_kernel");
  }
  hipLaunchKernelGGL(append_copy_kernel, dim3((unsigned)((items + kThreads - 1) / kThreads)), dim3(kThreads), 0, s, p);
  int rc = sc_launch_status("append_copy_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(append_finalize_kernel, dim3((t->batch + 63) / 64), dim3(64), 0, s, p);
  return sc_launch_status("append_finalize_kernel");
}

extern "C" int sc_tier_dequant(const ScTierDesc* t, int32_t first, int32_t count, void* k_out, void* v_out,
                               void* stream) {
  if (!t) return sc_fail(SC_ERR_INVALID, "sc_tier_dequant: null tier");
  if (count <= 0) return SC_OK;
  if (first < 0 || first + count > t->max_blocks) return sc_fail(SC_ERR_INVALID, "block range outside capacity");
  if (!k_out || !v_out) return sc_fail(SC_ERR_INVALID, "null outputs");
  DequantParams p;
  p.t = *t;
  p.first = first;
  p.count = count;
  p.k_out = (h16*)k_out;
  p.v_out = (h16*)v_out;
  const long n = (long)t->batch * t->kv_heads * count * t->block_size * t->head_dim;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, p);
  return sc_launch_status("dequant_kernel");
}
