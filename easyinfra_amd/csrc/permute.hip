// Row gather into expert-contiguous order, and the weighted top-k combine.
//
// gather  replaces send_hidden_states = h[send_indices] (moe_all2all.py:351).
// combine replaces _all2all_chunk_output_compute (moe_all2all.py:291-307):
//   out = zeros[T,H]; out.index_add_(0, token, y * w[:,None])
// as a token-major gather-reduce through the inverse permutation ``pos``: each
// output row is written once, accumulated in fp32 in slot order, no atomics, so
// the result is deterministic run to run.  Optional extras fused into the same
// pass: split-K partial outputs of the down projection (summed before weighting),
// and the shared-expert output (weight 1.0, moe_all2all.py:535-537).
#include "common.h"
#include "kernels.h"

namespace eimoe {

__device__ __forceinline__ void load8(const void* base, int dtype, long long off, float* v) {
  if (dtype == kBF16) {
    const u32x4_t q = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(base) + off);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(q[i] << 16);
      v[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
    }
  } else {
    const f32x4_t a = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + off);
    const f32x4_t b = *reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + off + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
}

__device__ __forceinline__ void store8(void* base, int dtype, long long off, const float* v) {
  if (dtype == kBF16) {
    u32x4_t q;
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = pack_bf16x2(v[2 * i], v[2 * i + 1]);
    *reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(base) + off) = q;
  } else {
    f32x4_t a, b;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = v[i];
      b[i] = v[4 + i];
    }
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(base) + off) = a;
    *reinterpret_cast<f32x4_t*>(static_cast<float*>(base) + off + 4) = b;
  }
}

__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ x, int row_bytes,
                                                          const int32_t* __restrict__ rows,
                                                          const int32_t* __restrict__ num_rows, int max_rows,
                                                          uint8_t* __restrict__ xs) {
  const int n = min(*num_rows, max_rows);
  const int cpr = row_bytes / 16;
  const long long total = static_cast<long long>(n) * cpr;
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<long long>(gridDim.x) * 256) {
    const int r = static_cast<int>(i / cpr);
    const int c = static_cast<int>(i % cpr);
    const long long src = static_cast<long long>(rows[r]) * row_bytes + c * 16;
    *reinterpret_cast<u32x4_t*>(xs + static_cast<long long>(r) * row_bytes + c * 16) =
        *reinterpret_cast<const u32x4_t*>(x + src);
  }
}

hipError_t launch_gather_rows(const void* x, int row_bytes, const int32_t* rows, const int32_t* num_rows,
                              int max_rows, void* xs, hipStream_t s) {
  const long long total = static_cast<long long>(max_rows) * (row_bytes / 16);
  long long blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                     static_cast<const uint8_t*>(x), row_bytes, rows, num_rows, max_rows, static_cast<uint8_t*>(xs));
  return hipGetLastError();
}

__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ y, int y_dtype, int n_split,
                                                      long long split_stride, const int32_t* __restrict__ pos,
                                                      const float* __restrict__ w, int T, int k, int H,
                                                      const void* __restrict__ shared_y, int shared_dtype,
                                                      int shared_n, void* __restrict__ out, int out_dtype) {
  const int cpr = H / 8;
  const long long total = static_cast<long long>(T) * cpr;
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<long long>(gridDim.x) * 256) {
    const int t = static_cast<int>(i / cpr);
    const int h = static_cast<int>(i % cpr) * 8;
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.f;
    for (int j = 0; j < k; ++j) {
      const int p = pos[static_cast<long long>(t) * k + j];
      if (p < 0) continue;
      const float wj = w[static_cast<long long>(t) * k + j];
      float ys[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) ys[q] = 0.f;
      for (int s = 0; s < n_split; ++s) {
        float v[8];
        load8(y, y_dtype, s * split_stride + static_cast<long long>(p) * H + h, v);
#pragma unroll
        for (int q = 0; q < 8; ++q) ys[q] += v[q];
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += wj * ys[q];
    }
    if (shared_y) {
      float ys[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) ys[q] = 0.f;
      for (int s = 0; s < shared_n; ++s) {
        float v[8];
        load8(shared_y, shared_dtype, (static_cast<long long>(s) * T + t) * H + h, v);
#pragma unroll
        for (int q = 0; q < 8; ++q) ys[q] += v[q];
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += ys[q];
    }
    store8(out, out_dtype, static_cast<long long>(t) * H + h, acc);
  }
}

// Non-temporal load of 8 consecutive elements (the partial planes are read once).
__device__ __forceinline__ void load8_nt(const void* base, int dtype, long long off, float* v) {
  if (dtype == kBF16) {
    const u32x4_t q =
        __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(base) + off));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(q[i] << 16);
      v[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
    }
  } else {
    const f32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + off));
    const f32x4_t b =
        __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(static_cast<const float*>(base) + off + 4));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[4 + i] = b[i];
    }
  }
}

// combine_kernel with the slot count K and the split count NS fixed (K * NS <= 8): a token's row
// positions and weights are loaded first, then every partial-plane row it sums, all in flight
// together with the non-temporal hint, instead of a chain of dependent loads per slot.  The sums
// run in the same order as combine_kernel's (per slot the split planes in plane order, then the
// weighted slots in slot order, then the shared planes), so the results are bit-identical.
// Used for batches of up to kCombineFixedMaxT tokens, where the chain of round trips is the cost
// (cold, one box: Mixtral-8x7B 64 tokens with two planes 7.6 -> 6.6 us, Qwen3-30B-A3B 32-expert share
// 32 / 256 tokens 8.1 / 8.4 -> 6.4 / 6.7 us); on large batches the planes were just written and
// partly sit in the last-level cache, which the non-temporal loads give up (Mixtral-8x7B 8192
// tokens 58 -> 62 us for one plane, DeepSeek-V2-Lite 4096 tokens 47 -> 52 us), so they keep the loop.
template <int K, int NS>
__global__ __launch_bounds__(256) void combine_fixed_kernel(const void* __restrict__ y, int y_dtype,
                                                            long long split_stride, const int32_t* __restrict__ pos,
                                                            const float* __restrict__ w, int T, int H,
                                                            const void* __restrict__ shared_y, int shared_dtype,
                                                            int shared_n, void* __restrict__ out, int out_dtype) {
  const int cpr = H / 8;
  const long long total = static_cast<long long>(T) * cpr;
  for (long long i = blockIdx.x * 256ll + threadIdx.x; i < total; i += static_cast<long long>(gridDim.x) * 256) {
    const int t = static_cast<int>(i / cpr);
    const int h = static_cast<int>(i % cpr) * 8;
    int p[K];
    float wj[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      p[j] = pos[static_cast<long long>(t) * K + j];
      wj[j] = w[static_cast<long long>(t) * K + j];
    }
    float v[K][NS][8];
#pragma unroll
    for (int j = 0; j < K; ++j)
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (p[j] >= 0) {
          load8_nt(y, y_dtype, s * split_stride + static_cast<long long>(p[j]) * H + h, v[j][s]);
        } else {
#pragma unroll
          for (int q = 0; q < 8; ++q) v[j][s][q] = 0.f;
        }
      }
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      if (p[j] < 0) continue;
      float ys[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) ys[q] = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int q = 0; q < 8; ++q) ys[q] += v[j][s][q];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += wj[j] * ys[q];
    }
    if (shared_y) {
      float ys[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) ys[q] = 0.f;
      for (int s = 0; s < shared_n; ++s) {
        float v2[8];
        load8_nt(shared_y, shared_dtype, (static_cast<long long>(s) * T + t) * H + h, v2);
#pragma unroll
        for (int q = 0; q < 8; ++q) ys[q] += v2[q];
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) acc[q] += ys[q];
    }
    store8(out, out_dtype, static_cast<long long>(t) * H + h, acc);
  }
}

hipError_t launch_combine(const void* y, int y_dtype, int n_split, long long split_stride, const int32_t* pos,
                          const float* w, int T, int k, int H, const void* shared_y, int shared_dtype, int shared_n,
                          void* out, int out_dtype, hipStream_t s) {
  const long long total = static_cast<long long>(T) * (H / 8);
  long long blocks = (total + 255) / 256;
  if (blocks > 16384) blocks = 16384;
  if (blocks < 1) blocks = 1;
  const dim3 g(static_cast<unsigned>(blocks));
  constexpr int kCombineFixedMaxT = 512;
#define EIMOE_CF(K, NS)                                                                                            \
  if (T <= kCombineFixedMaxT && k == K && n_split == NS) {                                                        \
    hipLaunchKernelGGL((combine_fixed_kernel<K, NS>), g, dim3(256), 0, s, y, y_dtype, split_stride, pos, w, T, H, \
                       shared_y, shared_dtype, shared_n, out, out_dtype);                                         \
    return hipGetLastError();                                                                                     \
  }
  EIMOE_CF(1, 1) EIMOE_CF(1, 2) EIMOE_CF(1, 4) EIMOE_CF(2, 1) EIMOE_CF(2, 2) EIMOE_CF(2, 4)
  EIMOE_CF(4, 1) EIMOE_CF(4, 2) EIMOE_CF(6, 1) EIMOE_CF(8, 1)
#undef EIMOE_CF
  hipLaunchKernelGGL(combine_kernel, g, dim3(256), 0, s, y, y_dtype, n_split, split_stride, pos, w, T, k, H, shared_y,
                     shared_dtype, shared_n, out, out_dtype);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------- decode: down + combine
// For a few routed pairs per expert (a decode step where each resident expert serves about one
// token) the down projection and the weighted combine run as one kernel, per (token, block of
// kDcCols output columns): for each of the token's slots in slot order whose expert is resident,
// y = h[pos] . W_d[e][cols]^T (h = hi + lo when the precise mode keeps a second term), then
// out[t, cols] = sum_j w_j * y_j (+ the shared-expert planes), fp32 throughout.  No y round trip
// through memory and no combine launch.  The 256 threads are kDcCols columns x kDcSlices K slices;
// each slice's partial sums are added in slice order through LDS (deterministic).
constexpr int kDcCols = 16;
constexpr int kDcSlices = 16;

__global__ __launch_bounds__(kDcCols* kDcSlices) void down_combine_kernel(
    const uint16_t* __restrict__ h, const uint16_t* __restrict__ h_lo, const uint16_t* __restrict__ w_down, int I,
    int H, const int32_t* __restrict__ ids, const float* __restrict__ wts, const int32_t* __restrict__ pos, int k,
    int e_lo, const void* __restrict__ shared_y, int shared_dtype, int shared_n, int T, void* __restrict__ out,
    int out_dtype) {
  __shared__ float part[kDcSlices][kDcCols];
  const int c = threadIdx.x % kDcCols;
  const int q = threadIdx.x / kDcCols;
  const int t = blockIdx.y;
  const int col = blockIdx.x * kDcCols + c;
  const int per = I / kDcSlices;          // a multiple of 8
  const int k0 = q * per;
  float acc = 0.f;
  for (int j = 0; j < k; ++j) {
    const int p = pos[static_cast<long long>(t) * k + j];
    if (p < 0) continue;                  // expert not resident on this GPU
    const int e = ids[static_cast<long long>(t) * k + j] - e_lo;
    const uint16_t* wr = w_down + (static_cast<long long>(e) * H + col) * I + k0;
    const uint16_t* hr = h + static_cast<long long>(p) * I + k0;
    const uint16_t* lr = h_lo ? h_lo + static_cast<long long>(p) * I + k0 : nullptr;
    // 8 partial sums, one per bf16 position of a 16-byte vector, so consecutive vectors' loads
    // and FMAs are independent and several loads stay in flight
    float d[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
    for (int kk = 0; kk < per; kk += 8) {
      const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(wr + kk);
      const u32x4_t hv = *reinterpret_cast<const u32x4_t*>(hr + kk);
      u32x4_t lv = {0u, 0u, 0u, 0u};
      if (lr) lv = *reinterpret_cast<const u32x4_t*>(lr + kk);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float h0 = __uint_as_float(hv[i] << 16) + __uint_as_float(lv[i] << 16);
        const float h1 = __uint_as_float(hv[i] & 0xffff0000u) + __uint_as_float(lv[i] & 0xffff0000u);
        d[2 * i] = fmaf(h0, __uint_as_float(wv[i] << 16), d[2 * i]);
        d[2 * i + 1] = fmaf(h1, __uint_as_float(wv[i] & 0xffff0000u), d[2 * i + 1]);
      }
    }
    part[q][c] = ((d[0] + d[1]) + (d[2] + d[3])) + ((d[4] + d[5]) + (d[6] + d[7]));
    __syncthreads();
    if (q == 0) {
      float y = 0.f;
#pragma unroll
      for (int s = 0; s < kDcSlices; ++s) y += part[s][c];
      acc += wts[static_cast<long long>(t) * k + j] * y;
    }
    __syncthreads();
  }
  if (q != 0) return;
  if (shared_y) {
    for (int s = 0; s < shared_n; ++s) {
      const long long off = (static_cast<long long>(s) * T + t) * H + col;
      acc += shared_dtype == kBF16 ? bf16_to_f32(static_cast<const uint16_t*>(shared_y)[off])
                                   : static_cast<const float*>(shared_y)[off];
    }
  }
  const long long o = static_cast<long long>(t) * H + col;
  if (out_dtype == kBF16) static_cast<uint16_t*>(out)[o] = f32_to_bf16(acc);
  else static_cast<float*>(out)[o] = acc;
}

bool down_combine_supported(int H, int I) { return H % kDcCols == 0 && I % (8 * kDcSlices) == 0; }

hipError_t launch_down_combine(const void* h, const void* h_lo, const void* w_down, int I, int H, const int32_t* ids,
                               const float* w, const int32_t* pos, int T, int k, int e_lo, const void* shared_y,
                               int shared_dtype, int shared_n, void* out, int out_dtype, hipStream_t s) {
  if (!down_combine_supported(H, I) || T < 1 || T > 65535) return hipErrorInvalidValue;
  hipLaunchKernelGGL(down_combine_kernel, dim3(H / kDcCols, T), dim3(kDcCols * kDcSlices), 0, s,
                     static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(h_lo),
                     static_cast<const uint16_t*>(w_down), I, H, ids, w, pos, k, e_lo, shared_y, shared_dtype,
                     shared_n, T, out, out_dtype);
  return hipGetLastError();
}

}  // namespace eimoe
