// INT8 symmetric quantisation (gfx950).
//
// Bit-exact restatement of spectral_cache.py:452-516:
//   absmax = max(max|x|, 1e-8f);  scale = absmax / 127.0f   (IEEE fp32 division)
//   code   = rint(x / scale)                                (IEEE division, ties to even)
// The reference keeps only round(x/scale)*scale and [min, max]; the codes
// and scales are stored here, and [min, max] is returned for API parity.
#include <math.h>

#include "sc_common.h"

namespace {

constexpr int kThreads = 256;

__device__ float block_reduce_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, red[i]);
  return r;
}

// One workgroup per group of n elements (PER_HEAD / PER_TENSOR).
__global__ __launch_bounds__(kThreads) void quant_group_kernel(const float* x, long n, int8_t* codes, float* scales,
                                                               float* minmax) {
  __shared__ float red[16];
  const long g = blockIdx.x;
  const float* xg = x + g * n;
  float am = 0.f, mn = INFINITY, mx = -INFINITY;
  for (long i = threadIdx.x; i < n; i += kThreads) {
    const float v = xg[i];
    am = fmaxf(am, fabsf(v));
    mn = fminf(mn, v);
    mx = fmaxf(mx, v);
  }
  const float gam = block_reduce_max(am, red);
  const float gmn = -block_reduce_max(-mn, red);
  const float gmx = block_reduce_max(mx, red);
  const float scale = fmaxf(gam, 1e-8f) / 127.0f;
  int8_t* cg = codes + g * n;
  for (long i = threadIdx.x; i < n; i += kThreads) cg[i] = (int8_t)(int)rintf(xg[i] / scale);
  if (threadIdx.x == 0) {
    scales[g] = scale;
    if (minmax) {
      minmax[2 * g] = gmn;
      minmax[2 * g + 1] = gmx;
    }
  }
}

// One wavefront per row (PER_ROW); minmax per group is reduced separately.
__global__ __launch_bounds__(kThreads) void quant_row_kernel(const float* x, long nrows, long cols, int8_t* codes,
                                                             float* scales) {
  const long row = (long)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= nrows) return;
  const int l = threadIdx.x & 63;
  const float* xr = x + row * cols;
  float am = 0.f;
  for (long i = l; i < cols; i += 64) am = fmaxf(am, fabsf(xr[i]));
  am = wave_max(am);
  const float scale = fmaxf(am, 1e-8f) / 127.0f;
  for (long i = l; i < cols; i += 64) codes[row * cols + i] = (int8_t)(int)rintf(xr[i] / scale);
  if (l == 0) scales[row] = scale;
}

__global__ __launch_bounds__(kThreads) void minmax_group_kernel(const float* x, long n, float* minmax) {
  __shared__ float red[16];
  const float* xg = x + (long)blockIdx.x * n;
  float mn = INFINITY, mx = -INFINITY;
  for (long i = threadIdx.x; i < n; i += kThreads) {
    mn = fminf(mn, xg[i]);
    mx = fmaxf(mx, xg[i]);
  }
  const float gmn = -block_reduce_max(-mn, red);
  const float gmx = block_reduce_max(mx, red);
  if (threadIdx.x == 0) {
    minmax[2 * blockIdx.x] = gmn;
    minmax[2 * blockIdx.x + 1] = gmx;
  }
}

}  // namespace

extern "C" int sc_quantize_int8(const float* x, int64_t groups, int64_t rows, int64_t cols, int32_t granularity,
                                int8_t* codes, float* scales, float* minmax, void* stream) {
  if (groups < 0 || rows < 0 || cols < 0) return sc_fail(SC_ERR_INVALID, "negative sizes");
  if (groups == 0 || rows == 0 || cols == 0) return SC_OK;
  if (!x || !codes || !scales) return sc_fail(SC_ERR_INVALID, "null pointer");
  hipStream_t s = (hipStream_t)stream;
  switch (granularity) {
    case SC_QUANT_PER_HEAD:
      hipLaunchKernelGGL(quant_group_kernel, dim3((unsigned)groups), dim3(kThreads), 0, s, x, (long)(rows * cols),
                         codes, scales, minmax);
      return sc_launch_status("quant_group_kernel");
    case SC_QUANT_PER_TENSOR:
      if (minmax) {
        // [groups][2] per-group minmax is not defined for one global scale;
        // write the global [min, max] once.
        hipLaunchKernelGGL(quant_group_kernel, dim3(1), dim3(kThreads), 0, s, x, (long)(groups * rows * cols), codes,
                           scales, minmax);
      } else {
        hipLaunchKernelGGL(quant_group_kernel, dim3(1), dim3(kThreads), 0, s, x, (long)(groups * rows * cols), codes,
                           scales, (float*)nullptr);
      }
      return sc_launch_status("quant_group_kernel");
    case SC_QUANT_PER_ROW: {
      const long nrows = (long)(groups * rows);
      hipLaunchKernelGGL(quant_row_kernel, dim3((unsigned)((nrows + 3) / 4)), dim3(kThreads), 0, s, x, nrows,
                         (long)cols, codes, scales);
      int rc = sc_launch_status("quant_row_kernel");
      if (rc || !minmax) return rc;
      hipLaunchKernelGGL(minmax_group_kernel, dim3((unsigned)groups), dim3(kThreads), 0, s, x, (long)(rows * cols),
                         minmax);
      return sc_launch_status("minmax_group_kernel");
    }
    default:
      return sc_fail(SC_ERR_INVALID, "bad granularity %d", granularity);
  }
}
