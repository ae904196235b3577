// K4a RMSNorm (+ fused residual add) and the SwiGLU gate for the TinyLlama
// forward (vllmlite/model.py:17-23, 96, 116-119). fp32, one wavefront per row:
// the rows are short (d_model 384) and many, so a row never needs more than
// one wave and no LDS.
#include "vl_common.h"

namespace {

template <int VPL>  // values per lane held in registers (dim <= 64 * VPL)
__global__ void __launch_bounds__(64) rms_norm_kernel(float* __restrict__ out,
                                                      float* __restrict__ residual,
                                                      const float* __restrict__ x,
                                                      const float* __restrict__ w, int64_t rows,
                                                      int dim, float eps) {
  const int lane = threadIdx.x;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    float v[VPL];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      float a = 0.f;
      if (c < dim) {
        a = x[r * dim + c];
        if (residual) {
          a = residual[r * dim + c] + a;
          residual[r * dim + c] = a;
        }
      }
      v[i] = a;
      ss += a * a;
    }
    ss = wave_sum(ss);
    // numpy: mean -> float32 sum / n; + eps (float32); sqrt; x / rms * w
    const float var = ss / (float)dim;
    const float rms = sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int c = lane + 64 * i;
      if (c < dim) out[r * dim + c] = (v[i] / rms) * w[c];
    }
  }
}

// silu(g) * u with each step rounded like numpy's float32 elementwise ops
__device__ __forceinline__ float silu_times(float g, float u) {
#pragma clang fp contract(off)
  const float s = g / (1.0f + expf(-g));
  return s * u;
}

// out[t, j] = silu(gu[t, j]) * gu[t, dff + j], silu(x) = x / (1 + exp(-x))
__global__ void __launch_bounds__(256) silu_mul_kernel(float* __restrict__ out,
                                                       const float* __restrict__ gu,
                                                       int64_t rows, int dff) {
  const int64_t n = rows * dff;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / dff;
    const int j = (int)(i - r * dff);
    const float g = gu[r * 2 * dff + j];
    const float u = gu[r * 2 * dff + dff + j];
    out[i] = silu_times(g, u);
  }
}

}  // namespace

extern "C" int vl_rms_norm(float* out, float* residual, const float* x, const float* weight,
                           int64_t rows, int dim, float eps, void* stream) {
  VL_CHECK_ARG(rows >= 0 && dim > 0 && dim <= 64 * 16, "bad shape (dim <= 1024)");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(out && x && weight, "null pointer");
  const int grid = (int)(rows < 65536 ? rows : 65536);
  hipStream_t st = (hipStream_t)stream;
  if (dim <= 64 * 4)
    rms_norm_kernel<4><<<grid, 64, 0, st>>>(out, residual, x, weight, rows, dim, eps);
  else if (dim <= 64 * 8)
    rms_norm_kernel<8><<<grid, 64, 0, st>>>(out, residual, x, weight, rows, dim, eps);
  else
    rms_norm_kernel<16><<<grid, 64, 0, st>>>(out, residual, x, weight, rows, dim, eps);
  VL_CHECK_LAUNCH();
  return VL_OK;
}

extern "C" int vl_silu_mul(float* out, const float* gate_up, int64_t rows, int d_ff,
                           void* stream) {
  VL_CHECK_ARG(rows >= 0 && d_ff > 0, "bad shape");
  if (rows == 0) return VL_OK;
  VL_CHECK_ARG(out && gate_up, "null pointer");
  const int64_t n = rows * d_ff;
  const int grid = (int)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
  silu_mul_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(out, gate_up, rows, d_ff);
  VL_CHECK_LAUNCH();
  return VL_OK;
}
