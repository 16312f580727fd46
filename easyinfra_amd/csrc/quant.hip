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

// Any row length or alignment: two passes over the row.
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

// Rows held in registers: 16-byte loads (8 bf16 or 4 fp32 per lane and vector), one
// HBM read per element, then the block absmax and the quantised bytes from the same
// registers.  V = 16-byte vectors per lane (row length <= V * 256 vectors).
template <int V, bool BF16>
__global__ __launch_bounds__(256) void quantize_rows_reg_kernel(const void* __restrict__ x, long long rows, int cols,
                                                                uint8_t* __restrict__ q, float* __restrict__ scale) {
  constexpr int kPer = BF16 ? 8 : 4;   // elements per 16-byte vector
  __shared__ float s_red[4];
  const int tid = threadIdx.x;
  const int nvec = cols / kPer;
  for (long long r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + r * cols * (BF16 ? 2 : 4));
    float f[V][kPer];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int i = tid + j * 256;
      const uint4 u = i < nvec ? src[i] : make_uint4(0u, 0u, 0u, 0u);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if constexpr (BF16) {
          f[j][2 * t] = __uint_as_float(w[t] << 16);
          f[j][2 * t + 1] = __uint_as_float(w[t] & 0xffff0000u);
        } else {
          f[j][t] = __uint_as_float(w[t]);
        }
      }
    }
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < V; ++j)
#pragma unroll
      for (int t = 0; t < kPer; ++t) amax = fmaxf(amax, fabsf(f[j][t]));
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    if ((tid & 63) == 0) s_red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    __syncthreads();
    const float s = amax > 0.f ? amax / 448.0f : 1.0f;
    if (tid == 0) scale[r] = s;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int i = tid + j * 256;
      if (i >= nvec) continue;
      uint32_t o[kPer / 4];
#pragma unroll
      for (int t = 0; t < kPer / 4; ++t) {
        int w = __builtin_amdgcn_cvt_pk_fp8_f32(f[j][4 * t] / s, f[j][4 * t + 1] / s, 0, false);
        w = __builtin_amdgcn_cvt_pk_fp8_f32(f[j][4 * t + 2] / s, f[j][4 * t + 3] / s, w, true);
        o[t] = static_cast<uint32_t>(w);
      }
      if constexpr (BF16)
        reinterpret_cast<uint2*>(q + r * cols)[i] = make_uint2(o[0], o[1]);
      else
        reinterpret_cast<uint32_t*>(q + r * cols)[i] = o[0];
    }
  }
}

template <bool BF16>
void launch_quantize_reg(int v, dim3 grid, hipStream_t s, const void* x, long long rows, int cols, uint8_t* q,
                         float* scale) {
  switch (v) {
#define EIMOE_QV(N) \
  case N: hipLaunchKernelGGL((quantize_rows_reg_kernel<N, BF16>), grid, dim3(256), 0, s, x, rows, cols, q, scale); break;
    EIMOE_QV(1) EIMOE_QV(2) EIMOE_QV(3) EIMOE_QV(4) EIMOE_QV(5) EIMOE_QV(6) EIMOE_QV(7) EIMOE_QV(8)
#undef EIMOE_QV
  }
}

hipError_t launch_quantize_rows_fp8(const void* x, int dtype, long long rows, int cols, uint8_t* q, float* scale,
                                    hipStream_t s) {
  long long blocks = rows < 16384 ? rows : 16384;
  if (blocks < 1) blocks = 1;
  const dim3 grid(static_cast<unsigned>(blocks));
  const int per = dtype == kBF16 ? 8 : 4;
  const int v = (cols / per + 255) / 256;
  // register path: 16-byte aligned rows of at most 8 vectors per lane (16384 bf16 / 8192 fp32 elements)
  if (cols > 0 && cols % per == 0 && v <= 8 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(q) & 7) == 0) {
    if (dtype == kBF16) launch_quantize_reg<true>(v, grid, s, x, rows, cols, q, scale);
    else launch_quantize_reg<false>(v, grid, s, x, rows, cols, q, scale);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(quantize_rows_fp8_kernel, grid, dim3(256), 0, s, x, dtype, rows, cols, q, scale);
  return hipGetLastError();
}

}  // namespace eimoe
