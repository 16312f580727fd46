// Shared device helpers for the gfx950 (CDNA4) MoE kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eimoe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef int i32x8_t __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Hardware facts of MI355X / gfx950 used for launch shaping.
constexpr int kNumXcd = 8;          // XCDs; workgroups are dispatched round-robin over them
constexpr int kNumCu = 256;         // compute units
constexpr int kLdsBytes = 160 * 1024;

enum DType : int { kF32 = 0, kBF16 = 1, kFP8 = 2 };

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 -> bf16 with v_cvt_pk_bf16_f32 (the kernels run with fp32
// denormals preserved and round-to-nearest-even).  It gives the bits of the integer recipe
// (u + 0x7fff + ((u >> 16) & 1)) >> 16, NaNs quieted to (u >> 16) | 0x40, on every one of
// the 2^32 fp32 patterns (compared exhaustively on gfx950), in one instruction per pair.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return static_cast<uint16_t>(pack_bf16x2(f, 0.f)); }

// Four OCP e4m3fn bytes -> four bf16 (exact: e4m3 values are representable in bf16).
// The fp32 produced by the hardware converter has a zero low half, so truncation is exact.
__device__ __forceinline__ u32x2_t fp8x4_to_bf16x4(uint32_t w) {
  f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  u32x2_t r;
  r[0] = (__float_as_uint(lo[0]) >> 16) | (__float_as_uint(lo[1]) & 0xffff0000u);
  r[1] = (__float_as_uint(hi[0]) >> 16) | (__float_as_uint(hi[1]) & 0xffff0000u);
  return r;
}

// silu(g) = g * sigmoid(g) with the hardware reciprocal (v_rcp_f32, <= 1 ulp) in place of an
// IEEE division: the division compiles to ~12 VALU instructions (div_scale x2, rcp, five FMAs,
// div_fmas, div_fixup), and the 256x256 SiLU epilogue forms 64 of these per lane, which measured
// ~5 us of a ~60-140 us tile.  Large |g| behave as the division does: exp(-g) = inf gives
// rcp(inf) = 0 and g * 0 = -0; exp(-g) = 0 gives g.
__device__ __forceinline__ float silu_f32(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g));
}

// Raw buffer resource over [base, base + bytes): loads past the end return zero.
constexpr int kBufDword3 = 0x00020000;  // gfx9 raw buffer resource word 3
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, long long bytes) {
  const uint32_t n = bytes <= 0 ? 0u : (bytes >= 0xffffffffll ? 0xffffffffu : static_cast<uint32_t>(bytes));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(n),
                                           kBufDword3);
}

// A wave-uniform value, taken from the first lane.  Buffer windows and tile coordinates are
// uniform by construction, but where they derive from values read out of LDS (the tile
// decode) the compiler cannot prove it: it then keeps them in VGPRs and wraps every buffer
// instruction in a readfirstlane loop (measured: 8 such loops per K slab in the 256x256
// e4m3 kernel).  Taking them from the first lane once, at the tile's start, keeps them in SGPRs.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ long long uniform(long long v) {
  const uint64_t u = static_cast<uint64_t>(v);
  // each half as uint32_t: the builtin returns int, and a sign-extended low half would set
  // every bit of the high half (a pointer with address bit 31 set would become 0xffffffff...)
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u)));
  return static_cast<long long>((static_cast<uint64_t>(hi) << 32) | lo);
}
template <class T>
__device__ __forceinline__ T* uniform(T* p) {
  return reinterpret_cast<T*>(uniform(reinterpret_cast<long long>(p)));
}

// Wave-wide inclusive prefix sum (64 lanes).
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

template <int N>
struct Log2 {
  static constexpr int value = 1 + Log2<N / 2>::value;
};
template <>
struct Log2<1> {
  static constexpr int value = 0;
};

}  // namespace eimoe
