// sc_decode_attn_noalloc: decode attention with the partial records in a
// library-owned device array instead of a caller workspace, for callers
// that cannot allocate device memory.  No counterpart in the reference.
//
// `scratch` below is a host-side stand-in for the device array: host code
// never passes it to a kernel or a copy.  The array's device address on the
// current GPU comes from hipGetSymbolAddress, taken once per device on the
// first call made with that device current, and that address is what the
// decode kernels receive as their record buffer.  Every unit of the partial
// kernel writes its whole record before the combine kernel reads it, so the
// array needs no clearing between calls; calls that overlap on one GPU share
// it and race.
#include <mutex>

#include "sc_common.h"

namespace {

static __device__ __align__(256) char scratch[SC_DECODE_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  SC_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices)
    return sc_fail(SC_ERR_UNSUPPORTED, "sc_decode_attn_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    SC_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return sc_fail(SC_ERR_HIP, "hipGetSymbolAddress returned a null address for the decode scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SC_OK;
}

}  // namespace

extern "C" int sc_decode_attn_noalloc(const ScDecodeArgs* args, void* stream) {
  size_t need = 0;
  int rc = sc_decode_workspace_size(args, &need);
  if (rc) return rc;
  if (need > SC_DECODE_SCRATCH_BYTES)
    return sc_fail(SC_ERR_WORKSPACE,
                   "sc_decode_attn_noalloc: this call needs %zu bytes of partial records, more than the "
                   "built-in scratch of %u bytes; use sc_decode_attn with a workspace",
                   need, (unsigned)SC_DECODE_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  return sc_decode_attn(args, ws, SC_DECODE_SCRATCH_BYTES, stream);
}
