// Query rotation of a decode or prefill step (gfx950): one launch for what
// the reference's apply_rotary_pos_emb (integration.py:428-465) does with
// five elementwise tensor ops when its decode caller rotates the queries
// (integration.py:610-613):
//   out = x * cos + rotate_half(x) * sin,  rotate_half(x) = (-x2, x1)
// in fp16 elementwise arithmetic: each product and the sum rounded to fp16,
// in that order.  fp32 holds 24 >= 2 * 11 + 2 significand bits, so an fp16
// product or sum computed in fp32 and rounded to fp16 equals the directly
// rounded fp16 operation: packed fp16 multiplies and adds give the same bits
// as the tensor ops.  Contraction is off so that no product is fused into
// the sum.
#include "sc_common.h"

namespace {

constexpr int kThreads = 256;

struct RopeParams {
  const h16* x;
  long xb, xh, xt;  // element strides of x [batch][heads][tokens][D]
  const h16* cos;
  const h16* sin;
  long cb, ct;      // element strides of cos/sin [batch][tokens][D] (cb = 0: shared by the batch)
  h16* out;         // [batch][heads][tokens][D], contiguous
  int B, H, T, D;
};

typedef _Float16 half8v __attribute__((ext_vector_type(8)));

// One work item = 8 consecutive elements (16 bytes) of one output row.
__global__ __launch_bounds__(kThreads) void rope_rotate_kernel(RopeParams p) {
#pragma clang fp contract(off)
  const int cpr = p.D / 8;  // chunks per row
  const long idx = (long)blockIdx.x * kThreads + threadIdx.x;
  const long rows = (long)p.B * p.H * p.T;
  if (idx >= rows * cpr) return;
  const long row = idx / cpr;
  const int c = (int)(idx % cpr);
  const int t = (int)(row % p.T);
  const int h = (int)((row / p.T) % p.H);
  const int b = (int)(row / ((long)p.T * p.H));
  const h16* xr = p.x + b * p.xb + h * p.xh + t * p.xt;
  const int d = 8 * c, half = p.D / 2;
  const bool first = d < half;
  const half8v xv = *reinterpret_cast<const half8v*>(xr + d);
  const half8v pv = *reinterpret_cast<const half8v*>(xr + (first ? d + half : d - half));
  const long cs = b * p.cb + (long)t * p.ct + d;
  const half8v cv = *reinterpret_cast<const half8v*>(p.cos + cs);
  const half8v sv = *reinterpret_cast<const half8v*>(p.sin + cs);
  const half8v rot = first ? -pv : pv;
  const half8v m1 = xv * cv;
  const half8v m2 = rot * sv;
  *reinterpret_cast<half8v*>(p.out + row * p.D + d) = m1 + m2;
}

}  // namespace

extern "C" int sc_rope_rotate(const void* x, int64_t x_stride_b, int64_t x_stride_h, int64_t x_stride_t,
                              const void* cos, const void* sin, int64_t cs_stride_b, int64_t cs_stride_t,
                              int32_t batch, int32_t heads, int32_t tokens, int32_t head_dim, void* out,
                              void* stream) {
  if (batch < 0 || heads < 0 || tokens < 0) return sc_fail(SC_ERR_INVALID, "sc_rope_rotate: negative extent");
  if (head_dim < 16 || head_dim > 256 || head_dim % 16)
    return sc_fail(SC_ERR_UNSUPPORTED, "sc_rope_rotate: head_dim %d must be a multiple of 16 in [16, 256]",
                   head_dim);
  if ((long)batch * heads * tokens == 0) return SC_OK;
  if (!x || !cos || !sin || !out) return sc_fail(SC_ERR_INVALID, "sc_rope_rotate: null pointer");
  if (((uintptr_t)x & 15) || ((uintptr_t)cos & 15) || ((uintptr_t)sin & 15) || ((uintptr_t)out & 15) ||
      (x_stride_b & 7) || (x_stride_h & 7) || (x_stride_t & 7) || (cs_stride_b & 7) || (cs_stride_t & 7))
    return sc_fail(SC_ERR_INVALID, "sc_rope_rotate: rows must be 16-byte aligned (strides multiples of 8)");
  RopeParams p;
  p.x = (const h16*)x;
  p.xb = x_stride_b;
  p.xh = x_stride_h;
  p.xt = x_stride_t;
  p.cos = (const h16*)cos;
  p.sin = (const h16*)sin;
  p.cb = cs_stride_b;
  p.ct = cs_stride_t;
  p.out = (h16*)out;
  p.B = batch;
  p.H = heads;
  p.T = tokens;
  p.D = head_dim;
  const long items = (long)batch * heads * tokens * (head_dim / 8);
  hipLaunchKernelGGL(rope_rotate_kernel, dim3((unsigned)((items + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     (hipStream_t)stream, p);
  return sc_launch_status("rope_rotate_kernel");
}
