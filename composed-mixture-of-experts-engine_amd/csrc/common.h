// Shared device helpers for the gfx950 MoE hot-path kernels.
//
// Element types crossing the C ABI are identified by moe_dtype codes
// (MOE_F32 = 0, MOE_BF16 = 1).  bf16 values are handled as raw 16-bit
// patterns; conversion to float is exact and conversion from float rounds to
// nearest-even (the same rounding torch uses for .to(torch.bfloat16)).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdio>
#include <string>

#include "../../include/moe_mi355.h"

namespace moe {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

// float -> bf16, round to nearest even, NaN stays NaN: gfx950's v_cvt_pk_bf16_f32 (bit-identical to the
// integer rounding u + 0x7fff + ((u >> 16) & 1) on every non-NaN input; checked exhaustively on the GPU).
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ float load_f(const void* p, int dt, int64_t i) {
  return dt == MOE_BF16 ? bf2f(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_f(void* p, int dt, int64_t i, float v) {
  if (dt == MOE_BF16)
    static_cast<uint16_t*>(p)[i] = f2bf(v);
  else
    static_cast<float*>(p)[i] = v;
}

// Pack two floats as two bf16 in one dword (low half = a), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{a, b}), bf16x2_t));
}

// Sum of two rows of 8 bf16 (one 16-byte word each) in fp32, rounded to bf16: the result of adding the two
// bf16 tensors (each pair is widened exactly, summed in fp32 and rounded to nearest even once).
__device__ __forceinline__ u32x4 add_bf16x8(const u32x4& v, const u32x4& a) {
  u32x4 r;
#pragma unroll
  for (int d = 0; d < 4; ++d)
    r[d] = pack2bf(__uint_as_float(v[d] << 16) + __uint_as_float(a[d] << 16),
                   __uint_as_float(v[d] & 0xffff0000u) + __uint_as_float(a[d] & 0xffff0000u));
  return r;
}

__device__ __forceinline__ f32x4 mfma16x16x32(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x16 mfma32x32x16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS operations (lgkmcnt(0)) but, unlike
// __syncthreads (whose fence also waits for every outstanding global load and store, vmcnt(0)), leaves global
// prefetches and stores in flight.  The empty asm statements keep the compiler from moving memory accesses
// across it.
__device__ __forceinline__ void lds_sync() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt((15) | (3 << 14) | (7 << 4));  // vmcnt, expcnt unconstrained; lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// Raw buffer descriptor over nbytes at base: loads at offsets past nbytes (or through a descriptor with
// no records) return zeros without touching memory.
typedef __amdgpu_buffer_rsrc_t buf_rsrc_t;
__device__ __forceinline__ buf_rsrc_t buf_rsrc(const void* base, int nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, nbytes, 0x00020000);
}
// Cache-policy operand of the buffer loads: sc1 makes a load read past this XCD's L2 (agent coherence).
constexpr int kPolicyCoherent = 16;

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

template <typename T>
__device__ __forceinline__ T wave_max(T v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Cross-lane moves inside each aligned row of 16 lanes by DPP (a VALU operand modifier: no LDS traffic,
// a few cycles of latency).  Step 0 pairs lane l with l^1 and step 1 with l^2 (quad permutes), step 2
// with 7-l inside each half row (row_half_mirror) and step 3 with 15-l (row_mirror): combining a value
// with its partner's at each step leaves the combination of all 16 lanes in every lane of the row, and
// for a commutative combine every lane holds bit-identical results.
template <int STEP>
__device__ __forceinline__ int row16_partner(int v) {
  constexpr int kCtrl = STEP == 0 ? 0xB1 : (STEP == 1 ? 0x4E : (STEP == 2 ? 0x141 : 0x140));
  return __builtin_amdgcn_update_dpp(v, v, kCtrl, 0xF, 0xF, false);
}
template <int STEP>
__device__ __forceinline__ float row16_partner(float v) {
  return __int_as_float(row16_partner<STEP>(__float_as_int(v)));
}

// Reductions inside each aligned group of 16 lanes.
__device__ __forceinline__ float row16_sum(float v) {
  v += row16_partner<0>(v);
  v += row16_partner<1>(v);
  v += row16_partner<2>(v);
  v += row16_partner<3>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, row16_partner<0>(v));
  v = fmaxf(v, row16_partner<1>(v));
  v = fmaxf(v, row16_partner<2>(v));
  v = fmaxf(v, row16_partner<3>(v));
  return v;
}

__device__ __forceinline__ bool better(float v, int e, float bv, int be) {
  return v > bv || (v == bv && e < be);
}

// Order-preserving map of a float to uint32: a larger float gets a larger key (-0 is folded into +0 so
// the two compare equal as floats do); every float's key is nonzero, so 0 can mark "no candidate".
// NaN must be mapped to -inf by the caller.
__device__ __forceinline__ uint32_t order_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float order_val(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Row-wide max / min of unsigned / signed 32-bit values (the DPP move folds into the max / min).
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, (uint32_t)row16_partner<0>((int)v));
  v = max(v, (uint32_t)row16_partner<1>((int)v));
  v = max(v, (uint32_t)row16_partner<2>((int)v));
  v = max(v, (uint32_t)row16_partner<3>((int)v));
  return v;
}
__device__ __forceinline__ int row16_min_i32(int v) {
  v = min(v, row16_partner<0>(v));
  v = min(v, row16_partner<1>(v));
  v = min(v, row16_partner<2>(v));
  v = min(v, row16_partner<3>(v));
  return v;
}

// Arg-max over each row of 16 lanes of (key, index): the larger key, the lower index on a tie.  Two
// mask-free passes: the row max of the keys, then the row min of the indices of the lanes holding it.
__device__ __forceinline__ void row16_argmax_key(uint32_t& bk, int& be) {
  const uint32_t w = row16_max_u32(bk);
  be = row16_min_i32(bk == w ? be : 0x7fffffff);
  bk = w;
}

inline int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

// ---- error reporting (host side) ----
void set_error(const char* fmt, ...);
int fail_arg(const char* fmt, ...);
int check_launch(const char* what);

// ---- e4m3 row quantization shared by the fp8 entry points (csrc/fp8.hip); row_limit (a device count, or
// null) bounds the rows quantized to min(rows, *row_limit) ----
int quant_rows_fp8(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld, void* dst, float* scale,
                   const int* row_limit, hipStream_t s);

// ---- optional per-kernel timing (host side; off unless moe_prof_enable(1)) ----
// Brackets one launch with two hipEvents recorded on the launch stream.
struct ProfScope {
  ProfScope(const char* name, hipStream_t s);
  ~ProfScope();
  int slot;
  hipStream_t stream;
};

#define MOE_LAUNCH(name, kernel, grid, block, shm, stream, ...)          \
  do {                                                                  \
    ::moe::ProfScope _moe_ps(name, stream);                             \
    hipLaunchKernelGGL(kernel, grid, block, shm, stream, __VA_ARGS__);  \
  } while (0)

}  // namespace moe
