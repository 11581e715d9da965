// Cold-block wire format (gfx950): pack blocks of one sequence out of the
// strided tier arrays into self-describing contiguous records, and unpack
// them back.  Layout: ScBlockHeader in include/spectral_hip.h.
//
// One workgroup per (block, KV head) copies that head's slice of every
// section with 16-byte vector accesses (4-byte ones for the per-head
// scalars); the workgroup of head 0 also writes the record header (pack).
// Unpack checks every header first (one thread per record) and copies only
// if all match.  Pure HBM traffic: every byte is read once and written once.
#include <stddef.h>

#include "sc_common.h"

namespace {

constexpr int kThreads = 256;
static_assert(sizeof(ScBlockHeader) == 64, "64-byte record header");

__host__ __device__ inline uint32_t align16(uint64_t x) { return (uint32_t)((x + 15) & ~(uint64_t)15); }

// Section sizes per KV head and record layout for a tier geometry.
struct Layout {
  uint32_t head_bytes[SC_BLOCK_SECTIONS];  // bytes of one head's slice (minmax: one of K, V)
  uint32_t offsets[SC_BLOCK_SECTIONS];     // from the record start
  uint32_t record_bytes;
};

__host__ __device__ inline Layout block_layout(const ScTierDesc& t) {
  Layout l;
  const uint32_t T = (uint32_t)t.block_size, D = (uint32_t)t.head_dim, H = (uint32_t)t.kv_heads;
  const uint32_t srows = t.granularity == SC_QUANT_PER_ROW ? T : 1;
  l.head_bytes[0] = T * (uint32_t)t.kp_keys;      // codes_k
  l.head_bytes[1] = (uint32_t)t.kp_values * T;    // codes_v
  l.head_bytes[2] = srows * 4;                    // scales_k
  l.head_bytes[3] = srows * 4;                    // scales_v
  l.head_bytes[4] = D * (uint32_t)t.kp_keys * 2;  // basis_k
  l.head_bytes[5] = D * (uint32_t)t.kp_values * 2;  // basis_v
  l.head_bytes[6] = 8;                            // minmax: [2][H][2] fp32
  l.head_bytes[7] = 4;                            // vnorm
  uint64_t off = sizeof(ScBlockHeader);
  for (int s = 0; s < SC_BLOCK_SECTIONS; ++s) {
    l.offsets[s] = align16(off);
    off = (uint64_t)l.offsets[s] + (uint64_t)l.head_bytes[s] * H * (s == 6 ? 2 : 1);
  }
  l.record_bytes = align16(off);
  return l;
}

struct WireParams {
  ScTierDesc t;
  Layout lay;
  int seq, first, n;
  char* rec;        // records (pack: written, unpack: read)
  int32_t* status;  // unpack only
};

// The nine pieces of one (head, block) slice: tier address, record address
// and length (sections 0-5, minmax K, minmax V, vnorm).
constexpr int kPieces = 9;
struct Pieces {
  char* tier[kPieces];
  char* rec[kPieces];
  uint32_t bytes[kPieces];
};

__device__ inline Pieces pieces(const WireParams& w, char* rec, int h, int j) {
  const ScTierDesc& t = w.t;
  const Layout& L = w.lay;
  const long bhj = ((long)w.seq * t.kv_heads + h) * t.max_blocks + j;
  const bool per_row = t.granularity == SC_QUANT_PER_ROW;
  Pieces q;
  q.tier[0] = (char*)(t.codes_k + bhj * t.block_size * t.kp_keys);
  q.tier[1] = (char*)(t.codes_v + bhj * t.kp_values * t.block_size);
  q.tier[2] = (char*)(t.scales_k + (per_row ? bhj * t.block_size : bhj));
  q.tier[3] = (char*)(t.scales_v + (per_row ? bhj * t.block_size : bhj));
  q.tier[4] = (char*)t.basis_k + bhj * t.head_dim * t.kp_keys * 2;
  q.tier[5] = (char*)t.basis_v + bhj * t.head_dim * t.kp_values * 2;
  q.tier[6] = (char*)(t.minmax_k + bhj * 2);
  q.tier[7] = (char*)(t.minmax_v + bhj * 2);
  q.tier[8] = (char*)(t.vnorm + bhj);
  for (int s = 0; s < 6; ++s) {
    q.rec[s] = rec + L.offsets[s] + (uint64_t)h * L.head_bytes[s];
    q.bytes[s] = L.head_bytes[s];
  }
  q.rec[6] = rec + L.offsets[6] + (uint64_t)h * 8;
  q.rec[7] = rec + L.offsets[6] + (uint64_t)t.kv_heads * 8 + (uint64_t)h * 8;
  q.rec[8] = rec + L.offsets[7] + (uint64_t)h * 4;
  q.bytes[6] = q.bytes[7] = 8;
  q.bytes[8] = 4;
  return q;
}

__device__ inline void copy_bytes(char* dst, const char* src, uint32_t bytes) {
  if ((bytes & 15) == 0 && (((uintptr_t)dst | (uintptr_t)src) & 15) == 0) {
    for (uint32_t i = threadIdx.x; i < bytes / 16; i += kThreads)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {  // per-head scalars: 4-byte words
    for (uint32_t i = threadIdx.x; i < bytes / 4; i += kThreads)
      reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(src)[i];
  }
}

__device__ inline void make_header(const WireParams& w, int j, ScBlockHeader& hd) {
  hd.magic = SC_BLOCK_MAGIC;
  hd.version = SC_BLOCK_VERSION;
  hd.header_bytes = (uint16_t)sizeof(ScBlockHeader);
  hd.record_bytes = w.lay.record_bytes;
  hd.kv_heads = (uint16_t)w.t.kv_heads;
  hd.head_dim = (uint16_t)w.t.head_dim;
  hd.block_size = (uint16_t)w.t.block_size;
  hd.k_keys = (uint16_t)w.t.k_keys;
  hd.k_values = (uint16_t)w.t.k_values;
  hd.kp_keys = (uint16_t)w.t.kp_keys;
  hd.kp_values = (uint16_t)w.t.kp_values;
  hd.granularity = (uint8_t)w.t.granularity;
  hd.reserved = 0;
  hd.start_position = j >= 0 ? w.t.block_start[(long)w.seq * w.t.max_blocks + j] : 0;
  for (int s = 0; s < SC_BLOCK_SECTIONS; ++s) hd.offsets[s] = w.lay.offsets[s];
}

__global__ __launch_bounds__(kThreads) void pack_kernel(WireParams w) {
  const int H = w.t.kv_heads;
  const int k = blockIdx.x / H, h = blockIdx.x % H, j = w.first + k;
  char* rec = w.rec + (uint64_t)k * w.lay.record_bytes;
  const Pieces q = pieces(w, rec, h, j);
  for (int i = 0; i < kPieces; ++i) copy_bytes(q.rec[i], q.tier[i], q.bytes[i]);
  if (h == 0 && threadIdx.x == 0) {
    ScBlockHeader hd;
    make_header(w, j, hd);
    const uint32_t* hw = reinterpret_cast<const uint32_t*>(&hd);
    for (int i = 0; i < (int)(sizeof(ScBlockHeader) / 4); ++i) reinterpret_cast<uint32_t*>(rec)[i] = hw[i];
  }
}

// The record's header against the tier geometry (every field but
// start_position, the offsets included, so a record of another layout is
// never copied).
__device__ inline bool header_ok(const WireParams& w, const char* rec) {
  ScBlockHeader want;
  make_header(w, -1, want);
  const uint32_t* a = reinterpret_cast<const uint32_t*>(rec);
  const uint32_t* b = reinterpret_cast<const uint32_t*>(&want);
  constexpr int kStart = offsetof(ScBlockHeader, start_position) / 4;
  bool ok = true;
  for (int i = 0; i < (int)(sizeof(ScBlockHeader) / 4); ++i) ok &= (i == kStart) || a[i] == b[i];
  return ok;
}

// One thread per record: any header that does not match sets *status.
__global__ __launch_bounds__(kThreads) void check_kernel(WireParams w) {
  const int k = blockIdx.x * kThreads + threadIdx.x;
  if (k < w.n && !header_ok(w, w.rec + (uint64_t)k * w.lay.record_bytes)) atomicExch(w.status, SC_ERR_INVALID);
}

// Runs after check_kernel on the same stream: copies nothing unless every
// record matched (all or nothing, so NCOLD never covers a slot left stale).
__global__ __launch_bounds__(kThreads) void unpack_kernel(WireParams w) {
  if (*w.status != 0) return;
  const int H = w.t.kv_heads;
  const int k = blockIdx.x / H, h = blockIdx.x % H, j = w.first + k;
  char* rec = w.rec + (uint64_t)k * w.lay.record_bytes;
  const Pieces q = pieces(w, rec, h, j);
  for (int i = 0; i < kPieces; ++i) copy_bytes(q.tier[i], q.rec[i], q.bytes[i]);
  if (h == 0 && threadIdx.x == 0) {
    w.t.block_start[(long)w.seq * w.t.max_blocks + j] = reinterpret_cast<const ScBlockHeader*>(rec)->start_position;
    atomicMax(w.t.counters + w.seq * SC_NCOUNTERS + SC_CNT_NCOLD, j + 1);
  }
}

__global__ void clear_status_kernel(int32_t* status) { *status = 0; }

int check_range(const ScTierDesc* t, int32_t seq, int32_t first, int32_t n, const void* buf, size_t bytes,
                const char* what) {
  if (!t) return sc_fail(SC_ERR_INVALID, "%s: null tier", what);
  if (seq < 0 || seq >= t->batch) return sc_fail(SC_ERR_INVALID, "%s: sequence %d outside [0, %d)", what, seq, t->batch);
  if (n < 0 || first < 0 || first + n > t->max_blocks)
    return sc_fail(SC_ERR_INVALID, "%s: blocks [%d, %d) outside capacity %d", what, first, first + n, t->max_blocks);
  if (t->kv_heads > 0xffff || t->head_dim > 0xffff || t->block_size > 0xffff)
    return sc_fail(SC_ERR_UNSUPPORTED, "%s: geometry does not fit the 16-bit header fields", what);
  const size_t need = (size_t)n * block_layout(*t).record_bytes;
  if (n > 0 && (!buf || ((uintptr_t)buf & 15)))
    return sc_fail(SC_ERR_INVALID, "%s: buffer must be non-null and 16-byte aligned", what);
  if (bytes < need) return sc_fail(SC_ERR_CAPACITY, "%s: buffer holds %zu bytes, %zu needed", what, bytes, need);
  return SC_OK;
}

}  // namespace

extern "C" size_t sc_block_record_bytes(const ScTierDesc* t) { return t ? block_layout(*t).record_bytes : 0; }

extern "C" int sc_tier_pack(const ScTierDesc* t, int32_t seq, int32_t first_block, int32_t n_blocks, void* dst,
                            size_t dst_bytes, void* stream) {
  int rc = check_range(t, seq, first_block, n_blocks, dst, dst_bytes, "sc_tier_pack");
  if (rc || n_blocks == 0) return rc;
  WireParams w;
  w.t = *t;
  w.lay = block_layout(*t);
  w.seq = seq;
  w.first = first_block;
  w.n = n_blocks;
  w.rec = (char*)dst;
  w.status = nullptr;
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)(n_blocks * t->kv_heads)), dim3(kThreads), 0, (hipStream_t)stream, w);
  return sc_launch_status("pack_kernel");
}

extern "C" int sc_tier_unpack(const ScTierDesc* t, int32_t seq, int32_t first_block, int32_t n_blocks,
                              const void* src, size_t src_bytes, int32_t* status, void* stream) {
  int rc = check_range(t, seq, first_block, n_blocks, src, src_bytes, "sc_tier_unpack");
  if (rc) return rc;
  if (!status) return sc_fail(SC_ERR_INVALID, "sc_tier_unpack: null status");
  hipLaunchKernelGGL(clear_status_kernel, dim3(1), dim3(1), 0, (hipStream_t)stream, status);
  rc = sc_launch_status("clear_status_kernel");
  if (rc || n_blocks == 0) return rc;
  WireParams w;
  w.t = *t;
  w.lay = block_layout(*t);
  w.seq = seq;
  w.first = first_block;
  w.n = n_blocks;
  w.rec = (char*)src;
  w.status = status;
  hipLaunchKernelGGL(check_kernel, dim3((unsigned)((n_blocks + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, w);
  rc = sc_launch_status("check_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(unpack_kernel, dim3((unsigned)(n_blocks * t->kv_heads)), dim3(kThreads), 0, (hipStream_t)stream,
                     w);
  return sc_launch_status("unpack_kernel");
}
