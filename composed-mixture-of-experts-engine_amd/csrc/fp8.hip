// e4m3 (OCP fp8) payloads of the expert FFN forward.
//
// Each row gets one fp32 scale, absmax / 448 (448 is the largest e4m3 value), and its elements are
// multiplied by inv = 448 / absmax (one division per row) in fp32 and rounded to nearest even by
// v_cvt_pk_fp8_f32.  A row whose absmax is below 2^-118 -- all-zero rows, and rows so small that 448 / absmax
// would overflow fp32 (it does below 448 / FLT_MAX ~ 1.3e-36), turning 0 * inv into NaN -- is treated as a
// zero row: scale 1, inv 1 (its elements, all below 2^-118, round to +-0).
//
// k_permute_fp8     the dispatch payload: each token row is quantized once and written to the rows of its
//                   slots (the rows k_permute fills) at one byte per element -- half the bytes of the bf16
//                   permute -- with its scale in sx[row].
// k_quant_rows_fp8  any [rows, cols] matrix (the expert weights once, the SwiGLU activations per forward).
//
// One wave per row: pass 1 takes the row's absmax, pass 2 quantizes 8 elements per lane and stores them as
// one 8-byte word.  bf16 rows of up to 16K elements stay in registers between the passes (one read of the
// row from memory); longer rows and fp32 rows are read twice.
#include "common.h"

namespace moe {

constexpr float kE4M3Max = 448.f;
constexpr float kQuantTiny = 0x1p-118f;  // smallest absmax quantized with its own scale: 448 / 2^-118 < FLT_MAX

__device__ __forceinline__ void row_scale(float amax, float& sc, float& inv) {
  const bool live = amax >= kQuantTiny;
  sc = live ? amax / kE4M3Max : 1.f;
  inv = live ? kE4M3Max / amax : 1.f;
}
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T>
__device__ __forceinline__ void q_load8(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void q_load8<uint16_t>(const uint16_t* p, float (&v)[8]) {
  const u32x4 a = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    v[2 * m] = __uint_as_float(a[m] << 16);
    v[2 * m + 1] = __uint_as_float(a[m] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void q_load8<float>(const float* p, float (&v)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    v[m] = a[m];
    v[4 + m] = b[m];
  }
}

template <typename T>
__device__ __forceinline__ void quant_row(const T* __restrict__ src, int cols, uint8_t* __restrict__ dst,
                                          float* __restrict__ scale, int lane) {
  float amax = 0.f;
  for (int c = lane * 8; c < cols; c += 512) {
    float v[8];
    q_load8<T>(src + c, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max(amax);
  float sc, inv;
  row_scale(amax, sc, inv);
  if (lane == 0) *scale = sc;
  for (int c = lane * 8; c < cols; c += 512) {
    float v[8];
    q_load8<T>(src + c, v);
    uint32_t lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0] * inv, v[1] * inv, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2] * inv, v[3] * inv, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4] * inv, v[5] * inv, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6] * inv, v[7] * inv, hi, true);
    __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(dst + c));
  }
}

// The same in one pass over memory for rows of at most 512 * NCH elements: the row is held in registers
// (NCH 16-byte words of bf16 per lane) between the absmax and the quantization.
template <int NCH>
__device__ __forceinline__ void quant_row_reg(const uint16_t* __restrict__ src, int cols, uint8_t* __restrict__ dst,
                                              float* __restrict__ scale, int lane) {
  u32x4 w[NCH];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane * 8 + 512 * j;
    w[j] = c < cols ? *reinterpret_cast<const u32x4*>(src + c) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int m = 0; m < 4; ++m)
      amax = fmaxf(amax, fmaxf(fabsf(__uint_as_float(w[j][m] << 16)), fabsf(__uint_as_float(w[j][m] & 0xffff0000u))));
  }
  amax = wave_max(amax);
  // the packed words are pinned here: otherwise the compiler keeps the first pass's unpacked floats for the
  // second pass (twice the registers of the row: one wave per SIMD at 32 words a lane)
#pragma unroll
  for (int j = 0; j < NCH; ++j) __asm__ volatile("" : "+v"(w[j]));
  float sc, inv;
  row_scale(amax, sc, inv);
  if (lane == 0) *scale = sc;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int c = lane * 8 + 512 * j;
    float v[8];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      v[2 * m] = __uint_as_float(w[j][m] << 16);
      v[2 * m + 1] = __uint_as_float(w[j][m] & 0xffff0000u);
    }
    uint32_t lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0] * inv, v[1] * inv, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2] * inv, v[3] * inv, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4] * inv, v[5] * inv, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6] * inv, v[7] * inv, hi, true);
    if (c < cols) __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(dst + c));
  }
}

__device__ __forceinline__ int q_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Rows quantized: the first `rows`, or the first min(rows, *row_limit) when row_limit is given (a device count,
// e.g. the rows the expert segments cover, offsets[E]).
__device__ __forceinline__ int64_t q_rows(int64_t rows, const int* __restrict__ row_limit) {
  return row_limit ? min(rows, (int64_t)max(*row_limit, 0)) : rows;
}

template <int NCH>
__global__ __launch_bounds__(256) void k_quant_rows_fp8_reg(const uint16_t* __restrict__ src, int64_t rows, int cols,
                                                           int64_t ld, uint8_t* __restrict__ dst,
                                                           float* __restrict__ scale,
                                                           const int* __restrict__ row_limit) {
  const int lane = threadIdx.x & 63;
  rows = q_rows(rows, row_limit);
  for (int64_t r = (int64_t)blockIdx.x * 4 + q_wave(); r < rows; r += (int64_t)gridDim.x * 4)
    quant_row_reg<NCH>(src + r * ld, cols, dst + r * cols, scale + r, lane);
}

template <typename T>
__global__ __launch_bounds__(256) void k_quant_rows_fp8(const T* __restrict__ src, int64_t rows, int cols, int64_t ld,
                                                       uint8_t* __restrict__ dst, float* __restrict__ scale,
                                                       const int* __restrict__ row_limit) {
  const int lane = threadIdx.x & 63;
  rows = q_rows(rows, row_limit);
  for (int64_t r = (int64_t)blockIdx.x * 4 + q_wave(); r < rows; r += (int64_t)gridDim.x * 4)
    quant_row<T>(src + r * ld, cols, dst + r * cols, scale + r, lane);
}

// The quantized dispatch payload, one wave per token: the token row is quantized once (absmax pass, then a
// conversion pass) and each 8-byte word goes to every row the token's slots hold (rows in [0, offsets[E])),
// with the row's scale.
template <typename T>
__global__ __launch_bounds__(256) void k_permute_fp8(const T* __restrict__ x, const int* __restrict__ slot_row,
                                                    const int* __restrict__ offsets, int E, int K, int H, int64_t N,
                                                    uint8_t* __restrict__ xq, float* __restrict__ sx) {
  const int lane = threadIdx.x & 63;
  const int live = offsets[E];
  for (int64_t t = (int64_t)blockIdx.x * 4 + q_wave(); t < N; t += (int64_t)gridDim.x * 4) {
    const T* src = x + t * H;
    float amax = 0.f;
    for (int c = lane * 8; c < H; c += 512) {
      float v[8];
      q_load8<T>(src + c, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = wave_max(amax);
    float sc, inv;
    row_scale(amax, sc, inv);
    for (int kw = 0; kw < K; kw += 64) {
      const int kn = min(K - kw, 64);
      const int mine = lane < kn ? slot_row[t * K + kw + lane] : -1;
      if (lane < kn && mine >= 0 && mine < live) sx[mine] = sc;
      for (int c = lane * 8; c < H; c += 512) {
        float v[8];
        q_load8<T>(src + c, v);
        uint32_t lo = 0, hi = 0;
        lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[0] * inv, v[1] * inv, lo, false);
        lo = __builtin_amdgcn_cvt_pk_fp8_f32(v[2] * inv, v[3] * inv, lo, true);
        hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[4] * inv, v[5] * inv, hi, false);
        hi = __builtin_amdgcn_cvt_pk_fp8_f32(v[6] * inv, v[7] * inv, hi, true);
        for (int k = 0; k < kn; ++k) {
          const int r = __builtin_amdgcn_readlane(mine, k);
          if (r >= 0 && r < live)
            __builtin_nontemporal_store(u32x2{lo, hi}, reinterpret_cast<u32x2*>(xq + (int64_t)r * H + c));
        }
      }
    }
  }
}

namespace {
bool al16q(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
unsigned q_blocks(int64_t rows) { return (unsigned)std::min<int64_t>(4096, std::max<int64_t>(1, (rows + 3) / 4)); }
}  // namespace

int quant_rows_fp8(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld, void* dst, float* scale,
                   const int* row_limit, hipStream_t s) {
  if (rows < 0 || cols < 16 || cols % 16 || ld < cols || ld % 8 || cols > INT32_MAX / 2 ||
      (src_dtype != MOE_BF16 && src_dtype != MOE_F32))
    return fail_arg("moe_quant_rows_fp8: bad arguments rows=%lld cols=%lld ld=%lld (need cols %% 16 == 0, ld >= cols, "
                    "ld %% 8 == 0, bf16 or fp32)", (long long)rows, (long long)cols, (long long)ld);
  if (rows == 0) return 0;
  if (!src || !dst || !scale || !al16q(src) || !al16q(dst)) return fail_arg("moe_quant_rows_fp8: null or misaligned pointer");
  if (src_dtype == MOE_BF16 && cols <= 32 * 512) {
    // one pass: the row in registers (8 to 32 words a lane)
    const auto* sp = static_cast<const uint16_t*>(src);
    auto* dp = static_cast<uint8_t*>(dst);
    if (cols <= 8 * 512)
      MOE_LAUNCH("k_quant_rows_fp8", k_quant_rows_fp8_reg<8>, dim3(q_blocks(rows)), dim3(256), 0, s, sp, rows,
                 (int)cols, ld, dp, scale, row_limit);
    else if (cols <= 16 * 512)
      MOE_LAUNCH("k_quant_rows_fp8", k_quant_rows_fp8_reg<16>, dim3(q_blocks(rows)), dim3(256), 0, s, sp, rows,
                 (int)cols, ld, dp, scale, row_limit);
    else
      MOE_LAUNCH("k_quant_rows_fp8", k_quant_rows_fp8_reg<32>, dim3(q_blocks(rows)), dim3(256), 0, s, sp, rows,
                 (int)cols, ld, dp, scale, row_limit);
  } else if (src_dtype == MOE_BF16)
    MOE_LAUNCH("k_quant_rows_fp8", k_quant_rows_fp8<uint16_t>, dim3(q_blocks(rows)), dim3(256), 0, s,
               static_cast<const uint16_t*>(src), rows, (int)cols, ld, static_cast<uint8_t*>(dst), scale, row_limit);
  else
    MOE_LAUNCH("k_quant_rows_fp8", k_quant_rows_fp8<float>, dim3(q_blocks(rows)), dim3(256), 0, s,
               static_cast<const float*>(src), rows, (int)cols, ld, static_cast<uint8_t*>(dst), scale, row_limit);
  return check_launch("moe_quant_rows_fp8");
}
}  // namespace moe

using namespace moe;

extern "C" int moe_quant_rows_fp8(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld, void* dst,
                                  float* scale, void* stream) {
  return quant_rows_fp8(src, src_dtype, rows, cols, ld, dst, scale, nullptr, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int moe_permute_fp8(const void* x, int x_dtype, const int32_t* slot_row, const int32_t* offsets, int64_t N,
                               int64_t K, int64_t E, int64_t H, void* xq, float* sx, void* stream) {
  if (E < 1 || K < 1 || N < 0 || H < 16 || H % 16 || H > INT32_MAX / 2 || (x_dtype != MOE_BF16 && x_dtype != MOE_F32))
    return fail_arg("moe_permute_fp8: bad arguments (need H %% 16 == 0, bf16 or fp32 x)");
  if (N == 0) return 0;
  if (!x || !slot_row || !offsets || !xq || !sx || !al16q(x) || !al16q(xq))
    return fail_arg("moe_permute_fp8: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == MOE_BF16)
    MOE_LAUNCH("k_permute_fp8", k_permute_fp8<uint16_t>, dim3(q_blocks(N)), dim3(256), 0, s,
               static_cast<const uint16_t*>(x), slot_row, offsets, (int)E, (int)K, (int)H, N,
               static_cast<uint8_t*>(xq), sx);
  else
    MOE_LAUNCH("k_permute_fp8", k_permute_fp8<float>, dim3(q_blocks(N)), dim3(256), 0, s, static_cast<const float*>(x),
               slot_row, offsets, (int)E, (int)K, (int)H, N, static_cast<uint8_t*>(xq), sx);
  return check_launch("moe_permute_fp8");
}
