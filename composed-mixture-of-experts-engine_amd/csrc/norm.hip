// RMSNorm in front of the router, for gfx950: the caller step before the routed path
// (moe-engine/pkg/models/moe.py L:63-86 RMSNorm, L:125-126 ToyMoEBlock: x + moe(norm(x))).
//
//   xn = ((x * rsqrt(mean_h(x^2) + eps)) * gamma).to(x.dtype)     (all arithmetic in fp32)
//
// k_rmsnorm_fwd     one wave per row: pass 1 sums the squares, pass 2 (the row is still in L1 / L2)
//                   scales and stores xn; rstd is kept for the backward.
// k_rmsnorm_route   the same with the router forward fused in (bf16 x and gate, E <= 16): pass 2 also
//                   forms the token's logits from the bf16-rounded xn (the values the router would read)
//                   against the gate staged in LDS, routes the token in registers (softmax, top-k,
//                   renormalisation; the semantics of the MFMA router kernels) and accumulates the block's
//                   statistics, which the last block folds (router_fin.h).  The hidden state is read from
//                   HBM once for both the norm and the logits.
// k_rmsnorm_bwd     one wave per row: dx = r (g - xhat mean_h(g xhat)), g = gamma * (dxn + dxn2), with the
//                   dgamma partial of each block accumulated per wave in LDS (fixed order, no atomics) and
//                   summed over blocks by k_rmsnorm_dgamma.
#include "common.h"
#include "router_fin.h"

namespace moe {

constexpr int kNormMaxH = 8192;  // the backward keeps four H-float dgamma rows in LDS

template <typename T>
__device__ __forceinline__ void nload8(const T* p, float (&f)[8]);
template <>
__device__ __forceinline__ void nload8<uint16_t>(const uint16_t* p, float (&f)[8]) {
  const u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = __uint_as_float(v[j] << 16);
    f[2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void nload8<float>(const float* p, float (&f)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = a[j];
    f[4 + j] = b[j];
  }
}
template <typename T>
__device__ __forceinline__ void nstore8(T* p, const float (&f)[8]);
template <>
__device__ __forceinline__ void nstore8<uint16_t>(uint16_t* p, const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = pack2bf(f[2 * j], f[2 * j + 1]);
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
template <>
__device__ __forceinline__ void nstore8<float>(float* p, const float (&f)[8]) {
  __builtin_nontemporal_store(f32x4{f[0], f[1], f[2], f[3]}, reinterpret_cast<f32x4*>(p));
  __builtin_nontemporal_store(f32x4{f[4], f[5], f[6], f[7]}, reinterpret_cast<f32x4*>(p + 4));
}
// The value a stored element takes when read back (bf16 rounding; identity for fp32).
template <typename T>
__device__ __forceinline__ float as_stored(float v);
template <>
__device__ __forceinline__ float as_stored<uint16_t>(float v) { return bf2f(f2bf(v)); }
template <>
__device__ __forceinline__ float as_stored<float>(float v) { return v; }

__device__ __forceinline__ int norm_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Sum of squares of one row in fp32: lane-strided 8-element chunks, then a fixed butterfly.
template <typename T>
__device__ __forceinline__ float row_sumsq(const T* __restrict__ row, int H, int lane) {
  float ss = 0.f;
  for (int h0 = lane * 8; h0 < H; h0 += 512) {
    float v[8];
    nload8<T>(row + h0, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  }
  return wave_sum(ss);
}

// ---------------------------------------------------------------------------
// Forward.
// ---------------------------------------------------------------------------
template <typename TX, typename TG>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(const TX* __restrict__ x, const TG* __restrict__ gamma,
                                                    float eps, int N, int H, TX* __restrict__ xn,
                                                    float* __restrict__ rstd) {
  const int lane = threadIdx.x & 63;
  for (int t = blockIdx.x * 4 + norm_wave(); t < N; t += gridDim.x * 4) {
    const TX* row = x + (int64_t)t * H;
    const float r = rsqrtf(row_sumsq<TX>(row, H, lane) / (float)H + eps);
    if (lane == 0) rstd[t] = r;
    for (int h0 = lane * 8; h0 < H; h0 += 512) {
      float v[8], gv[8], o[8];
      nload8<TX>(row + h0, v);
      nload8<TG>(gamma + h0, gv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (v[i] * r) * gv[i];
      nstore8<TX>(xn + (int64_t)t * H + h0, o);
    }
  }
}

// ---------------------------------------------------------------------------
// Forward with the router fused in (bf16 x, bf16 gate, E <= EP in {8, 16}).  Block = 4 waves, one token
// per wave at a time.  The gate [H, E] is staged in LDS padded to EP experts per row (16 or 32 bytes).
// ---------------------------------------------------------------------------
template <typename TG, int EP>
__global__ __launch_bounds__(256) void k_rmsnorm_route(
    const uint16_t* __restrict__ x, const TG* __restrict__ gamma, float eps, const uint16_t* __restrict__ wg,
    const float* __restrict__ bias, int N, int H, int E, int K, uint16_t* __restrict__ xn,
    float* __restrict__ rstd, int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt,
    float* __restrict__ logits_out, float* __restrict__ lse_out, int* __restrict__ part_cnt,
    float* __restrict__ part_p, float* __restrict__ part_z, unsigned* __restrict__ ticket, float aux_coef,
    float z_coef, int64_t* __restrict__ cnt_out, float* __restrict__ stats, float* __restrict__ aux_out,
    float* __restrict__ z_out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t nsm[];
  uint16_t* wl = reinterpret_cast<uint16_t*>(nsm);  // [H][EP] bf16, experts past E zero
  int* s_cnt = reinterpret_cast<int*>(nsm + (size_t)H * EP * 2);
  float(*s_p)[EP] = reinterpret_cast<float(*)[EP]>(s_cnt + EP);
  float* s_z = reinterpret_cast<float*>(s_p + 4);
  int* s_nf = reinterpret_cast<int*>(s_z + 4);
  int* s_last = s_nf + 4;
  float* s_fin = reinterpret_cast<float*>(s_last + 4);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = norm_wave();
  for (int i = tid; i < H * EP; i += 256) {
    const int h = i / EP, e = i % EP;
    wl[i] = e < E ? wg[(int64_t)h * E + e] : (uint16_t)0;
  }
  if (tid < EP) s_cnt[tid] = 0;
  __syncthreads();

  float pacc = 0.f;  // lane e < E: this wave's sum of p[t, e]
  float zacc = 0.f;
  int nfacc = 0;
  for (int t = blockIdx.x * 4 + wv; t < N; t += gridDim.x * 4) {
    const uint16_t* row = x + (int64_t)t * H;
    const float r = rsqrtf(row_sumsq<uint16_t>(row, H, lane) / (float)H + eps);
    if (lane == 0) rstd[t] = r;
    float acc[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) acc[e] = 0.f;
    for (int h0 = lane * 8; h0 < H; h0 += 512) {
      float v[8], gv[8], o[8];
      nload8<uint16_t>(row + h0, v);
      nload8<TG>(gamma + h0, gv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = as_stored<uint16_t>((v[i] * r) * gv[i]);
      nstore8<uint16_t>(xn + (int64_t)t * H + h0, o);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t* wr = wl + (h0 + i) * EP;
#pragma unroll
        for (int c = 0; c < EP; c += 8) {
          const u32x4 wq = *reinterpret_cast<const u32x4*>(wr + c);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[c + 2 * j] = fmaf(o[i], __uint_as_float(wq[j] << 16), acc[c + 2 * j]);
            acc[c + 2 * j + 1] = fmaf(o[i], __uint_as_float(wq[j] & 0xffff0000u), acc[c + 2 * j + 1]);
          }
        }
      }
    }
    // logits of the token in every lane: row sums by DPP, then across the four rows of the wave
    float lg[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      float v = row16_sum(acc[e]);
      v += __shfl_xor(v, 16);
      v += __shfl_xor(v, 32);
      if (bias != nullptr && e < E) v += bias[e];
      lg[e] = v;
    }
    // ---- routing (every lane holds the same values; lane e / lane k store) ----
    float mine = 0.f;
    int nf = 0;
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      if (e == lane) mine = lg[e];
      if (e < E && !isfinite(lg[e])) ++nf;
      if (lg[e] != lg[e]) lg[e] = -INFINITY;  // NaN never wins a top-k slot
      if (e >= E) lg[e] = -INFINITY;
    }
    if (lane < E) logits_out[(int64_t)t * E + lane] = mine;
    float m = lg[0];
#pragma unroll
    for (int e = 1; e < EP; ++e) m = fmaxf(m, lg[e]);
    float ex[EP], s = 0.f;
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      ex[e] = expf(lg[e] - m);
      s += ex[e];
    }
    const float inv = 1.f / s;
    const float lse = m + logf(s);
    if (lane == 0) lse_out[t] = lse;
    zacc += lse * lse;
    nfacc += nf;
    float pe = 0.f;
#pragma unroll
    for (int e = 0; e < EP; ++e)
      if (e == lane) pe = ex[e] * inv;
    pacc += pe;
    // top-k: K rounds of arg-max (larger logit, lower id on a tie) over the experts not taken yet
    uint32_t taken = 0;
    int my_e = 0;
    float my_p = 0.f, psum = 0.f;
    for (int rk = 0; rk < K; ++rk) {
      float bv = -INFINITY;
      int be = 0x7fffffff;
#pragma unroll
      for (int e = 0; e < EP; ++e) {
        const bool ok = e < E && !((taken >> e) & 1u) && better(lg[e], e, bv, be);
        bv = ok ? lg[e] : bv;
        be = ok ? e : be;
      }
      taken |= 1u << be;
      const float pv = expf(bv - m) * inv;
      psum += pv;
      my_e = rk == lane ? be : my_e;
      my_p = rk == lane ? pv : my_p;
    }
    const float rden = 1.f / fmaxf(psum, 1e-30f);
    if (lane < K) {
      idx_out[(int64_t)t * K + lane] = my_e;
      store_f(w_out, w_dt, (int64_t)t * K + lane, my_p * rden);
      atomicAdd(&s_cnt[my_e], 1);
    }
  }
  if (lane < EP) s_p[wv][lane] = pacc;
  if (lane == 0) {
    s_z[wv] = zacc;
    s_nf[wv] = nfacc;
  }
  __syncthreads();
  // ---- block partials (fixed order over the 4 waves), then the last block folds all of them ----
  if (tid < E) {
    const float p = ((s_p[0][tid] + s_p[1][tid]) + s_p[2][tid]) + s_p[3][tid];
    st_part(&part_cnt[(int64_t)blockIdx.x * E + tid], s_cnt[tid]);
    st_part(&part_p[(int64_t)blockIdx.x * E + tid], p);
  }
  if (tid == 0) {
    st_part(&part_z[2 * blockIdx.x], ((s_z[0] + s_z[1]) + s_z[2]) + s_z[3]);
    st_part(&part_z[2 * blockIdx.x + 1], (float)(s_nf[0] + s_nf[1] + s_nf[2] + s_nf[3]));
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    *s_last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!*s_last) return;
  router_finalize_block<256, true>(part_cnt, part_p, part_z, gridDim.x, N, E, K, aux_coef, z_coef, cnt_out, stats,
                                   aux_out, z_out, s_fin);
  if (tid == 0) *ticket = 0u;
}

// ---------------------------------------------------------------------------
// Backward.  Wave w of a block accumulates its rows' dgamma terms in LDS row w; the block's partial is the
// fixed-order sum of the four rows.
// ---------------------------------------------------------------------------
template <typename TX, typename TG>
__global__ __launch_bounds__(256) void k_rmsnorm_bwd(const TX* __restrict__ x, const TG* __restrict__ gamma,
                                                    const float* __restrict__ rstd, const TX* __restrict__ dxn,
                                                    const TX* __restrict__ dxn2, int N, int H,
                                                    TX* __restrict__ dx, float* __restrict__ part_dg) {
  extern __shared__ __attribute__((aligned(16))) float s_dg[];  // [4][H]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = norm_wave();
  float* dgw = s_dg + wv * H;
  for (int i = lane; i < H; i += 64) dgw[i] = 0.f;
  for (int t = blockIdx.x * 4 + wv; t < N; t += gridDim.x * 4) {
    const float r = rstd[t];
    const TX* xr = x + (int64_t)t * H;
    const TX* gr = dxn + (int64_t)t * H;
    const TX* gr2 = dxn2 ? dxn2 + (int64_t)t * H : nullptr;
    // pass 1: dot = sum_h g xhat, and dgamma += dxn_total * xhat
    float dot = 0.f;
    for (int h0 = lane * 8; h0 < H; h0 += 512) {
      float v[8], gd[8], gv[8];
      nload8<TX>(xr + h0, v);
      nload8<TX>(gr + h0, gd);
      if (gr2) {
        float g2[8];
        nload8<TX>(gr2 + h0, g2);
#pragma unroll
        for (int i = 0; i < 8; ++i) gd[i] += g2[i];
      }
      nload8<TG>(gamma + h0, gv);
      f32x4 d0 = *reinterpret_cast<f32x4*>(dgw + h0), d1 = *reinterpret_cast<f32x4*>(dgw + h0 + 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xh = v[i] * r;
        dot = fmaf(gv[i] * gd[i], xh, dot);
        if (i < 4) d0[i] = fmaf(gd[i], xh, d0[i]);
        else d1[i - 4] = fmaf(gd[i], xh, d1[i - 4]);
      }
      *reinterpret_cast<f32x4*>(dgw + h0) = d0;
      *reinterpret_cast<f32x4*>(dgw + h0 + 4) = d1;
    }
    const float c = wave_sum(dot) / (float)H;
    // pass 2: dx = r (g - xhat c)
    for (int h0 = lane * 8; h0 < H; h0 += 512) {
      float v[8], gd[8], gv[8], o[8];
      nload8<TX>(xr + h0, v);
      nload8<TX>(gr + h0, gd);
      if (gr2) {
        float g2[8];
        nload8<TX>(gr2 + h0, g2);
#pragma unroll
        for (int i = 0; i < 8; ++i) gd[i] += g2[i];
      }
      nload8<TG>(gamma + h0, gv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = r * (gv[i] * gd[i] - (v[i] * r) * c);
      nstore8<TX>(dx + (int64_t)t * H + h0, o);
    }
  }
  __syncthreads();
  for (int i = tid; i < H; i += 256)
    part_dg[(int64_t)blockIdx.x * H + i] = ((s_dg[i] + s_dg[H + i]) + s_dg[2 * H + i]) + s_dg[3 * H + i];
}

// dgamma[h] = sum over blocks of part_dg[b][h], blocks in order.
__global__ __launch_bounds__(256) void k_rmsnorm_dgamma(const float* __restrict__ part_dg, int nblk, int H,
                                                       void* __restrict__ dgamma, int g_dt) {
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float s = 0.f;
  int b = 0;
  for (; b + 8 <= nblk; b += 8) {  // eight loads in flight, summed in block order
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part_dg[(int64_t)(b + u) * H + h];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; b < nblk; ++b) s += part_dg[(int64_t)b * H + h];
  store_f(dgamma, g_dt, h, s);
}

namespace {

int norm_blocks(int64_t N) { return (int)std::min<int64_t>(2048, std::max<int64_t>(1, (N + 3) / 4)); }
// the backward writes one dgamma partial row per block: about two blocks per CU
int norm_bwd_blocks(int64_t N) { return (int)std::min<int64_t>(512, std::max<int64_t>(1, (N + 3) / 4)); }
// Dynamic LDS above the default limit needs the kernel's attribute raised once.
template <typename K>
int allow_lds(K kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return check_launch("hipFuncSetAttribute");
  return 0;
}
// the fused router-norm keeps the block count moderate (one partial set per block for the fold)
int norm_route_blocks(int64_t N) { return (int)std::min<int64_t>(512, std::max<int64_t>(1, (N + 7) / 8)); }
int norm_route_ep(int64_t E) { return E <= 8 ? 8 : 16; }
size_t norm_route_lds(int64_t H, int EP) {
  return (size_t)H * EP * 2 + EP * 4 + 4 * EP * 4 + 4 * 4 + 4 * 4 + 4 * 4 +
         (size_t)finalize_scratch_floats<256>() * 4;
}
bool norm_route_fits(int64_t H, int64_t E) { return E <= 16 && norm_route_lds(H, norm_route_ep(E)) <= 80 * 1024; }

bool al16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define MOE_NORM_DT(xdt, gdt, CALL)                                                             \
  do {                                                                                          \
    if (xdt == MOE_BF16 && gdt == MOE_F32) { using TX = uint16_t; using TG = float; CALL; }     \
    else if (xdt == MOE_BF16) { using TX = uint16_t; using TG = uint16_t; CALL; }               \
    else if (gdt == MOE_F32) { using TX = float; using TG = float; CALL; }                      \
    else { using TX = float; using TG = uint16_t; CALL; }                                       \
  } while (0)

int norm_check(const char* what, int64_t N, int64_t H, int x_dt, int g_dt) {
  if (N < 0 || H < 8 || H % 8 || H > kNormMaxH)
    return fail_arg("%s: bad shape N=%lld H=%lld (need H %% 8 == 0, 8 <= H <= %d)", what, (long long)N, (long long)H,
                    kNormMaxH);
  if ((x_dt != MOE_F32 && x_dt != MOE_BF16) || (g_dt != MOE_F32 && g_dt != MOE_BF16))
    return fail_arg("%s: unsupported dtype", what);
  return 0;
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" int moe_rmsnorm_fwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, float eps, int64_t N,
                               int64_t H, void* xn_out, float* rstd_out, void* stream) {
  if (int rc = norm_check("moe_rmsnorm_fwd", N, H, x_dtype, gamma_dtype)) return rc;
  if (N == 0) return 0;
  if (!x || !gamma || !xn_out || !rstd_out || !al16p(x) || !al16p(gamma) || !al16p(xn_out))
    return fail_arg("moe_rmsnorm_fwd: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  MOE_NORM_DT(x_dtype, gamma_dtype,
              MOE_LAUNCH("k_rmsnorm_fwd", (k_rmsnorm_fwd<TX, TG>), dim3(norm_blocks(N)), dim3(256), 0, s,
                         static_cast<const TX*>(x), static_cast<const TG*>(gamma), eps, (int)N, (int)H,
                         static_cast<TX*>(xn_out), rstd_out));
  return check_launch("moe_rmsnorm_fwd");
}

extern "C" size_t moe_rmsnorm_router_fwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype,
                                                   int wg_dtype) {
  if (N <= 0 || H <= 0 || E <= 0) return 0;
  const size_t fused = 256 + ((size_t)norm_route_blocks(N) * E * 8 + 255) / 256 * 256 +
                       ((size_t)norm_route_blocks(N) * 2 * 4 + 255) / 256 * 256;
  return std::max(fused, moe_router_fwd_workspace(N, H, E, K, x_dtype, wg_dtype));
}

extern "C" int moe_rmsnorm_router_fwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, float eps,
                                      const void* wg, int wg_dtype, const float* bias, int64_t N, int64_t H,
                                      int64_t E, int64_t K, void* xn_out, float* rstd_out, int64_t* idx_out,
                                      void* w_out, int w_dtype, float* logits_out, float* lse_out, int64_t* cnt_out,
                                      float* stats_out, float aux_coef, float z_coef, float* aux_out, float* z_out,
                                      void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = norm_check("moe_rmsnorm_router_fwd", N, H, x_dtype, gamma_dtype)) return rc;
  if (E < 1 || E > kMaxE || K < 1 || K > E || K > kMaxK)
    return fail_arg("moe_rmsnorm_router_fwd: bad shape E=%lld K=%lld", (long long)E, (long long)K);
  if (N == 0) return moe_router_fwd(xn_out, x_dtype, wg, wg_dtype, bias, 0, H, E, K, idx_out, w_out, w_dtype,
                                    logits_out, lse_out, cnt_out, stats_out, aux_coef, z_coef, aux_out, z_out,
                                    workspace, ws_bytes, stream);
  const bool fused = x_dtype == MOE_BF16 && wg_dtype == MOE_BF16 && norm_route_fits(H, E) && al16p(x) &&
                     al16p(gamma) && al16p(xn_out) && (w_dtype == MOE_F32 || w_dtype == MOE_BF16);
  if (!fused) {
    // the norm, then the router over its output (the streaming / MFMA router kernels)
    if (int rc = moe_rmsnorm_fwd(x, x_dtype, gamma, gamma_dtype, eps, N, H, xn_out, rstd_out, stream)) return rc;
    return moe_router_fwd(xn_out, x_dtype, wg, wg_dtype, bias, N, H, E, K, idx_out, w_out, w_dtype, logits_out,
                          lse_out, cnt_out, stats_out, aux_coef, z_coef, aux_out, z_out, workspace, ws_bytes, stream);
  }
  if (!wg || !idx_out || !w_out || !logits_out || !lse_out || !cnt_out || !stats_out || !rstd_out)
    return fail_arg("moe_rmsnorm_router_fwd: null pointer argument");
  const int nblk = norm_route_blocks(N);
  const size_t off_cnt = 256, off_p = off_cnt + ((size_t)nblk * E * 4 + 255) / 256 * 256,
               off_z = off_p + ((size_t)nblk * E * 4 + 255) / 256 * 256,
               total = off_z + ((size_t)nblk * 2 * 4 + 255) / 256 * 256;
  if (ws_bytes < total || !workspace)
    return set_error("moe_rmsnorm_router_fwd: workspace %zu < %zu bytes", ws_bytes, total), MOE_EWORKSPACE;
  // the completion counter is the first word of the workspace: zero on entry, left zero (as the router's)
  char* ws = static_cast<char*>(workspace);
  unsigned* ticket = reinterpret_cast<unsigned*>(ws);
  int* pc = reinterpret_cast<int*>(ws + off_cnt);
  float* pp = reinterpret_cast<float*>(ws + off_p);
  float* pz = reinterpret_cast<float*>(ws + off_z);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int EP = norm_route_ep(E);
  const size_t lds = norm_route_lds(H, EP);
#define MOE_NR(TGv, EPv)                                                                                            \
  if (int rc = allow_lds(k_rmsnorm_route<TGv, EPv>, lds)) return rc;                                                 \
  MOE_LAUNCH("k_rmsnorm_route", (k_rmsnorm_route<TGv, EPv>), dim3(nblk), dim3(256), lds, s,                         \
             static_cast<const uint16_t*>(x), static_cast<const TGv*>(gamma), eps, static_cast<const uint16_t*>(wg), \
             bias, (int)N, (int)H, (int)E, (int)K, static_cast<uint16_t*>(xn_out), rstd_out, idx_out, w_out,        \
             w_dtype, logits_out, lse_out, pc, pp, pz, ticket, aux_coef, z_coef, cnt_out, stats_out, aux_out, z_out)
  if (gamma_dtype == MOE_F32) {
    if (EP == 8) {
      MOE_NR(float, 8);
    } else {
      MOE_NR(float, 16);
    }
  } else {
    if (EP == 8) {
      MOE_NR(uint16_t, 8);
    } else {
      MOE_NR(uint16_t, 16);
    }
  }
#undef MOE_NR
  return check_launch("moe_rmsnorm_router_fwd");
}

extern "C" size_t moe_rmsnorm_bwd_workspace(int64_t N, int64_t H) {
  if (N <= 0 || H <= 0) return 0;
  return ((size_t)norm_bwd_blocks(N) * H * 4 + 255) / 256 * 256;
}

extern "C" int moe_rmsnorm_bwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, const float* rstd,
                               const void* dxn, const void* dxn2, int64_t N, int64_t H, void* dx_out,
                               void* dgamma_out, void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = norm_check("moe_rmsnorm_bwd", N, H, x_dtype, gamma_dtype)) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!gamma || !dgamma_out) return fail_arg("moe_rmsnorm_bwd: null pointer argument");
  if (N == 0) {
    MOE_LAUNCH("k_rmsnorm_dgamma", k_rmsnorm_dgamma, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, s,
               static_cast<const float*>(nullptr), 0, (int)H, dgamma_out, gamma_dtype);
    return check_launch("moe_rmsnorm_bwd");
  }
  if (!x || !rstd || !dxn || !dx_out || !al16p(x) || !al16p(gamma) || !al16p(dxn) || !al16p(dx_out) ||
      (dxn2 && !al16p(dxn2)))
    return fail_arg("moe_rmsnorm_bwd: null or misaligned pointer");
  const int nblk = norm_bwd_blocks(N);
  if (ws_bytes < moe_rmsnorm_bwd_workspace(N, H) || !workspace)
    return set_error("moe_rmsnorm_bwd: workspace too small"), MOE_EWORKSPACE;
  float* part = static_cast<float*>(workspace);
  const size_t lds = (size_t)4 * H * 4;
  MOE_NORM_DT(x_dtype, gamma_dtype, if (int rc = allow_lds(k_rmsnorm_bwd<TX, TG>, lds)) return rc);
  MOE_NORM_DT(x_dtype, gamma_dtype,
              MOE_LAUNCH("k_rmsnorm_bwd", (k_rmsnorm_bwd<TX, TG>), dim3(nblk), dim3(256), lds, s,
                         static_cast<const TX*>(x), static_cast<const TG*>(gamma), rstd, static_cast<const TX*>(dxn),
                         static_cast<const TX*>(dxn2), (int)N, (int)H, static_cast<TX*>(dx_out), part));
  if (int rc = check_launch("k_rmsnorm_bwd")) return rc;
  MOE_LAUNCH("k_rmsnorm_dgamma", k_rmsnorm_dgamma, dim3((unsigned)((H + 255) / 256)), dim3(256), 0, s, part, nblk,
             (int)H, dgamma_out, gamma_dtype);
  return check_launch("moe_rmsnorm_bwd");
}
