// Per-row fp8-e4m3 (OCP e4m3fn) quantisation with absmax/448 scales.
//
// Used for expert weights (one scale per output channel = per row of [E*N, K])
// and for per-token dynamic activation scales.  No counterpart in the reference:
// fused_moe.py:331-335 accepts fp8 tensors but maps them to a bf16 compute type
// and takes no scales.  q = rne_e4m3(x / s) with s = max|x| / 448 (s = 1 for an
// all-zero row); division and conversion are correctly rounded, so the bytes
// match torch's CPU cast bit for bit.
#include "common.h"
#include "kernels.h"

namespace eimoe {

__global__ __launch_bounds__(256) void quantize_rows_fp8_kernel(const void* __restrict__ x, int dtype, long long rows,
                                                                int cols, uint8_t* __restrict__ q,
                                                                float* __restrict__ scale) {
  __shared__ float s_red[4];
  const int tid = threadIdx.x;
  for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
    float amax = 0.f;
    for (int c = tid; c < cols; c += 256) {
      const float v = dtype == kBF16 ? bf16_to_f32(static_cast<const uint16_t*>(x)[r * cols + c])
                                     : static_cast<const float*>(x)[r * cols + c];
      amax = fmaxf(amax, fabsf(v));
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    if ((tid & 63) == 0) s_red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    const float s = amax > 0.f ? amax / 448.0f : 1.0f;
    if (tid == 0) scale[r] = s;
    for (int c = 2 * tid; c < cols; c += 512) {
      float v0, v1 = 0.f;
      if (dtype == kBF16) {
        v0 = bf16_to_f32(static_cast<const uint16_t*>(x)[r * cols + c]);
        if (c + 1 < cols) v1 = bf16_to_f32(static_cast<const uint16_t*>(x)[r * cols + c + 1]);
      } else {
        v0 = static_cast<const float*>(x)[r * cols + c];
        if (c + 1 < cols) v1 = static_cast<const float*>(x)[r * cols + c + 1];
      }
      const int packed = __builtin_amdgcn_cvt_pk_fp8_f32(v0 / s, v1 / s, 0, false);
      q[r * cols + c] = static_cast<uint8_t>(packed & 0xff);
      if (c + 1 < cols) q[r * cols + c + 1] = static_cast<uint8_t>((packed >> 8) & 0xff);
    }
  }
}

hipError_t launch_quantize_rows_fp8(const void* x, int dtype, long long rows, int cols, uint8_t* q, float* scale,
                                    hipStream_t s) {
  long long blocks = rows < 16384 ? rows : 16384;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(quantize_rows_fp8_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, x, dtype, rows,
                     cols, q, scale);
  return hipGetLastError();
}

}  // namespace eimoe
