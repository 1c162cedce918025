// RMSNorm in front of the router, for gfx950: the caller step before the routed path
// (moe-engine/pkg/models/moe.py L:63-86 RMSNorm, L:125-126 ToyMoEBlock: x + moe(norm(x))).
//
//   xn = ((x * rsqrt(mean_h(x^2) + eps)) * gamma).to(x.dtype)     (all arithmetic in fp32)
//
// Row layout.  One wave owns one row at a time.  Lane l holds the 8-element chunks c = l + 64 j of the row
// (elements 8c .. 8c+7, j < NCH; NCH = 1, 4, 8 or 16 as H <= 512, 2048, 4096, 8192) in registers, as
// 16-byte words read through a buffer descriptor over the row (chunks past H read as zero without a
// memory access).  The next row's chunk j is requested as soon as the current row's chunk j has been used
// for the last time, so a wave keeps one row in flight while it computes on the other with no second
// buffer.  Per-column operands (gamma, the packed gate) sit in LDS in the same lane-major order, so every
// LDS read of a wave covers 64 consecutive 16-byte words (conflict-free).
//
// k_rmsnorm_fwd     pass 1 sums the squares, pass 2 scales, rounds and stores xn.
// k_rmsnorm_route   the same with the router forward fused in (bf16 x and gate, E <= 16), two rows per wave:
//                   pass 2 also dots the bf16-rounded xn pairs (the values the router would read) with the
//                   gate (v_dot2_f32_bf16, fp32 accumulation); the wave's partial logits of both tokens are
//                   reduce-scattered over the lanes, gathered into one 16-lane row per token and routed
//                   there with DPP (softmax, top-k, renormalisation: the semantics of the MFMA router
//                   kernels); the last block folds the block statistics (router_fin.h).  The hidden state
//                   is read from HBM once for both the norm and the logits.
// k_rmsnorm_bwd<.., EP>  dx = r (g - xhat mean_h(g xhat)) with g = gamma * u, where u = dxn (+ dxn2)
//                   (EP = 0) or u = dxn + G wg^T (EP = 8/16: the router's gradient of xn formed in place from
//                   G = dL/dlogits, never written to HBM), u rounded to the storage type.  dgamma += u xhat
//                   is kept per lane in registers, folded over the block's waves in LDS and over blocks by
//                   k_rmsnorm_dgamma.
#include <type_traits>

#include "common.h"
#include "router_fin.h"

namespace moe {

constexpr int kNormMaxH = 8192;
constexpr int kNormStream = 2;  // buffer-load policy of rows read once: nt

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2bf(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// 16-byte words per 8-element chunk
template <typename T>
constexpr int chunk_words() { return (int)sizeof(T) / 2; }

template <typename T, int NCH>
struct RowFrag {
  u32x4 w[NCH * chunk_words<T>()];
};

template <typename T, int NCH>
__device__ __forceinline__ void frag_load(RowFrag<T, NCH>& f, buf_rsrc_t r, int j, int lane) {
  const int off = (lane + 64 * j) * 8 * (int)sizeof(T);
#pragma unroll
  for (int q = 0; q < chunk_words<T>(); ++q)
    f.w[j * chunk_words<T>() + q] =
        __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * q, 0, kNormStream));
}
template <typename T, int NCH>
__device__ __forceinline__ void frag_load_all(RowFrag<T, NCH>& f, buf_rsrc_t r, int lane) {
#pragma unroll
  for (int j = 0; j < NCH; ++j) frag_load(f, r, j, lane);
}
template <int NCH>
__device__ __forceinline__ void frag_get(const RowFrag<uint16_t, NCH>& f, int j, float (&v)[8]) {
  const u32x4 a = f.w[j];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    v[2 * m] = __uint_as_float(a[m] << 16);
    v[2 * m + 1] = __uint_as_float(a[m] & 0xffff0000u);
  }
}
template <int NCH>
__device__ __forceinline__ void frag_get(const RowFrag<float, NCH>& f, int j, float (&v)[8]) {
  const u32x4 a = f.w[2 * j], b = f.w[2 * j + 1];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    v[m] = __uint_as_float(a[m]);
    v[4 + m] = __uint_as_float(b[m]);
  }
}

// Chunk c of a row (8 elements at 8c): rounded to the storage type and stored (streaming); for bf16 the
// packed pairs are returned in pk (the exact values a reader of the row sees).
template <typename T>
__device__ __forceinline__ void chunk_store(T* row, int c, bool ok, const float (&o)[8], u32x4& pk) {
  if constexpr (std::is_same<T, uint16_t>::value) {
#pragma unroll
    for (int m = 0; m < 4; ++m) pk[m] = pack2bf(o[2 * m], o[2 * m + 1]);
    if (ok) __builtin_nontemporal_store(pk, reinterpret_cast<u32x4*>(row + 8 * c));
  } else {
    if (ok) {
      __builtin_nontemporal_store(f32x4{o[0], o[1], o[2], o[3]}, reinterpret_cast<f32x4*>(row + 8 * c));
      __builtin_nontemporal_store(f32x4{o[4], o[5], o[6], o[7]}, reinterpret_cast<f32x4*>(row + 8 * c + 4));
    }
  }
}

// gamma in LDS as fp32, lane-major: word (2 j + q) 64 + l holds gamma[8 (l + 64 j) + 4 q .. + 3] (zero past H)
template <typename TG, int NCH>
__device__ __forceinline__ void stage_gamma(f32x4* s_gam, const TG* __restrict__ gamma, int H, int tid, int nthr) {
  for (int i = tid; i < NCH * 128; i += nthr) {
    const int l = i & 63, q = (i >> 6) & 1, j = i >> 7;
    const int h0 = 8 * (l + 64 * j) + 4 * q;
    f32x4 g = {0.f, 0.f, 0.f, 0.f};
    if (h0 < H) {  // H % 8 == 0, so the four elements are all in range
      if constexpr (std::is_same<TG, float>::value) {
        g = *reinterpret_cast<const f32x4*>(gamma + h0);
      } else {
        const uint2 u = *reinterpret_cast<const uint2*>(gamma + h0);
        g = f32x4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                  __uint_as_float(u.y & 0xffff0000u)};
      }
    }
    s_gam[i] = g;
  }
}
template <int NCH>
__device__ __forceinline__ void gamma_get(const f32x4* s_gam, int j, int lane, float (&g)[8]) {
  const f32x4 a = s_gam[(2 * j) * 64 + lane], b = s_gam[(2 * j + 1) * 64 + lane];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    g[m] = a[m];
    g[4 + m] = b[m];
  }
}

__device__ __forceinline__ int norm_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Start of a row iteration: the LDS operands (gamma, the gate image) are re-read from LDS in every row
// rather than hoisted out of the row loop into registers (that would take NCH * 8 to 256 VGPRs a lane).
__device__ __forceinline__ void row_fence() { __asm__ volatile("" ::: "memory"); }
// End of a chunk.  The running sums are materialised here and no memory access crosses this point, so the
// compiler can neither hoist every chunk's LDS reads to the top of the row nor sink every chunk's products
// to its end (either keeps all chunks' operands live at once: hundreds of VGPRs a lane).
template <int N>
__device__ __forceinline__ void chunk_fence(float (&acc)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) __asm__ volatile("" : "+v"(acc[i]));
  __asm__ volatile("" ::: "memory");
}
__device__ __forceinline__ void chunk_fence() { __asm__ volatile("" ::: "memory"); }

// Cross-lane partner of each level of a 64-lane exchange: lanes 32, 16 and 8 apart, 7 - l inside 8 lanes,
// then 2 and 1 apart (the last four by DPP, no LDS traffic).
__device__ __forceinline__ float dpp_xor8(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), 0x128, 0xF, 0xF, false));
}
template <int LV>
__device__ __forceinline__ float lane_partner(float v) {
  if constexpr (LV == 0) return __shfl_xor(v, 32);
  else if constexpr (LV == 1) return __shfl_xor(v, 16);
  else if constexpr (LV == 2) return dpp_xor8(v);
  else if constexpr (LV == 3) return row16_partner<2>(v);
  else if constexpr (LV == 4) return row16_partner<1>(v);
  else return row16_partner<0>(v);
}
template <int LV>
__device__ __forceinline__ float rs_sum(float v) {
  if constexpr (LV > 5) return v;
  else return rs_sum<LV + 1>(v + lane_partner<LV>(v));
}
template <int LV, int NV>
__device__ __forceinline__ float rs_level(const float (&in)[NV], int lane) {
  if constexpr (NV == 1) {
    return rs_sum<LV>(in[0]);
  } else {
    // keep the half of the index range this lane's bit selects, add the partner's copy of it
    const bool hi = ((lane >> (5 - LV)) & 1) != 0;
    float out[NV / 2];
#pragma unroll
    for (int m = 0; m < NV / 2; ++m) {
      const float keep = hi ? in[NV / 2 + m] : in[m];
      const float send = hi ? in[m] : in[NV / 2 + m];
      out[m] = keep + lane_partner<LV>(send);
    }
    return rs_level<LV + 1, NV / 2>(out, lane);
  }
}
// Partial sums acc[NV] of every lane (NV a power of two <= 64) -> lane l returns the wave total of index
// l / (64 / NV).  Each exchange halves the index range a lane keeps, the lanes of a group then sum what is
// left: NV - 1 + 6 - log2(NV) cross-lane moves instead of 6 per index.
template <int NV>
__device__ __forceinline__ float wave_reduce_scatter(const float (&acc)[NV], int lane) {
  return rs_level<0, NV>(acc, lane);
}

// The gate [H, E] bf16 staged into LDS in the order the kernels read it (experts past E, rows past H zero):
//   forward  (pairs along h): word ((q NCH + j) 4 + m) 64 + l, dword k = (wg[h][4q+k], wg[h+1][4q+k]),
//            h = 8 (l + 64 j) + 2 m, q < EP / 4
//   backward (pairs along e): word ((q NCH + j) 8 + i) 64 + l, dword k = (wg[h][8q+2k], wg[h][8q+2k+1]),
//            h = 8 (l + 64 j) + i, q < EP / 8
// With E == EP (16-byte aligned rows) each gate row is read as EP / 8 16-byte words.
template <int EP>
__device__ __forceinline__ void gate_row(const uint16_t* __restrict__ wg, int h, int H, int E, u32x4 (&r)[EP / 8]) {
#pragma unroll
  for (int u = 0; u < EP / 8; ++u) {
    if (E == EP) {
      r[u] = h < H ? *reinterpret_cast<const u32x4*>(wg + (int64_t)h * EP + 8 * u) : u32x4{0u, 0u, 0u, 0u};
    } else {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int e0 = 8 * u + 2 * d;
        const uint32_t lo = (h < H && e0 < E) ? wg[(int64_t)h * E + e0] : 0u;
        const uint32_t hi = (h < H && e0 + 1 < E) ? wg[(int64_t)h * E + e0 + 1] : 0u;
        r[u][d] = lo | (hi << 16);
      }
    }
  }
}
template <int NCH, int EP>
__device__ __forceinline__ void stage_gate_fwd(u32x4* s_w, const uint16_t* __restrict__ wg, int H, int E, int tid,
                                               int nthr) {
  for (int P = tid; P < NCH * 256; P += nthr) {  // rows h = 2P and 2P + 1
    const int h = 2 * P, c = P >> 2, m = P & 3, l = c & 63, j = c >> 6;
    u32x4 ra[EP / 8], rb[EP / 8];
    gate_row<EP>(wg, h, H, E, ra);
    gate_row<EP>(wg, h + 1, H, E, rb);
#pragma unroll
    for (int q = 0; q < EP / 4; ++q) {  // experts 4q .. 4q+3 sit in dwords d0, d0 + 1 of word u
      const int u = q >> 1, d0 = 2 * (q & 1);
      u32x4 w;
      w[0] = (ra[u][d0] & 0xffffu) | (rb[u][d0] << 16);
      w[1] = (ra[u][d0] >> 16) | (rb[u][d0] & 0xffff0000u);
      w[2] = (ra[u][d0 + 1] & 0xffffu) | (rb[u][d0 + 1] << 16);
      w[3] = (ra[u][d0 + 1] >> 16) | (rb[u][d0 + 1] & 0xffff0000u);
      s_w[((q * NCH + j) * 4 + m) * 64 + l] = w;
    }
  }
}
template <int NCH, int EP>
__device__ __forceinline__ void stage_gate_bwd(u32x4* s_w, const uint16_t* __restrict__ wg, int H, int E, int tid,
                                               int nthr) {
  for (int h = tid; h < NCH * 512; h += nthr) {
    const int c = h >> 3, i = h & 7, l = c & 63, j = c >> 6;
    u32x4 r[EP / 8];
    gate_row<EP>(wg, h, H, E, r);
#pragma unroll
    for (int q = 0; q < EP / 8; ++q) s_w[((q * NCH + j) * 8 + i) * 64 + l] = r[q];
  }
}

// Sum over the wave in a fixed order, returned as a wave-uniform value: row sums by DPP, the four rows
// combined by row broadcasts into lane 63 (no LDS round trips).
__device__ __forceinline__ float wave_total(float v) {
  v = row16_sum(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum of squares of a row held as a fragment, over the wave (the same order in every kernel).
template <typename T, int NCH>
__device__ __forceinline__ float frag_sumsq(const RowFrag<T, NCH>& f) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    float v[8];
    frag_get(f, j, v);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
  }
  return wave_total(ss);
}

// ---------------------------------------------------------------------------
// Forward.
// ---------------------------------------------------------------------------
struct NormFwdArgs {
  const void* x;
  const void* gamma;
  float eps;
  int N, H;
  void* xn;
  float* rstd;
  // router (k_rmsnorm_route)
  const uint16_t* wg;  // gate [H, E] bf16
  const float* bias;
  int E, K;
  int64_t* idx;
  void* w;
  int w_dt;
  float* logits;
  float* lse;
  int* part_cnt;
  float* part_p;
  float* part_z;
  unsigned* ticket;
  float aux_coef, z_coef;
  int64_t* cnt;
  float* stats;
  float* aux;
  float* z;
};

template <int NCH>
constexpr size_t norm_fwd_lds() { return (size_t)NCH * 2048; }

template <typename TX, typename TG, int NCH>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(NormFwdArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t nsm[];
  f32x4* s_gam = reinterpret_cast<f32x4*>(nsm);  // [NCH * 2][64]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = norm_wave();
  const int N = a.N, H = a.H;
  const TX* __restrict__ x = static_cast<const TX*>(a.x);
  TX* __restrict__ xn = static_cast<TX*>(a.xn);
  const int rowbytes = H * (int)sizeof(TX);
  const int nwt = gridDim.x * 4;
  int t = blockIdx.x * 4 + wv;
  RowFrag<TX, NCH> f;  // the first row is requested before the LDS staging, whose latency it then overlaps
  if (t < N) frag_load_all(f, buf_rsrc(x + (int64_t)t * H, rowbytes), lane);
  stage_gamma<TG, NCH>(s_gam, static_cast<const TG*>(a.gamma), H, tid, 256);
  __syncthreads();
  for (; t < N; t += nwt) {
    row_fence();
    const int tn = t + nwt;
    const buf_rsrc_t rn = buf_rsrc(x + (int64_t)tn * H, tn < N ? rowbytes : 0);
    const float r = rsqrtf(frag_sumsq(f) / (float)H + a.eps);
    if (lane == 0) a.rstd[t] = r;
    TX* orow = xn + (int64_t)t * H;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float v[8], g[8], o[8];
      frag_get(f, j, v);
      gamma_get<NCH>(s_gam, j, lane, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = (v[i] * r) * g[i];
      const int c = lane + 64 * j;
      u32x4 pk;
      chunk_store<TX>(orow, c, 8 * c < H, o, pk);
      frag_load(f, rn, j, lane);  // the next row's chunk j into the registers just freed
      chunk_fence();
    }
  }
}

// Forward with the router fused in (bf16 x and gate, E <= EP in {8, 16}).  One block per CU (the gate image
// fills most of the LDS).  Each wave takes R rows at a time, t_r = t0 + r * stride: one LDS read of the gate
// serves all R rows' dot products and one reduce-scatter + routing pass serves all R tokens (token r is
// routed by lanes 32 r .. 32 r + 31 for R = 2, by all lanes for R = 1, in the first 16-lane row of those).
// R = 2 with 8 waves a block, R = 1 with 16 (half the row registers, twice the waves).
template <int R>
constexpr int route_waves() { return R == 2 ? 8 : 16; }
template <int NCH, int EP, int R>
constexpr size_t norm_route_lds() {
  constexpr int NWV = route_waves<R>();
  return (size_t)NCH * 2048 + (size_t)EP * NCH * 1024 +
         (EP + NWV * EP + 2 * NWV + 4 + finalize_scratch_floats<NWV * 64>()) * 4;
}

template <typename TG, int NCH, int EP, int R>
__global__ __launch_bounds__(route_waves<R>() * 64) void k_rmsnorm_route(NormFwdArgs a) {
  constexpr int NWV = route_waves<R>();
  constexpr int NT = NWV * 64;
  constexpr int NV = R * EP;  // (token, expert) partial sums of a lane
  extern __shared__ __attribute__((aligned(16))) uint8_t nsm[];
  f32x4* s_gam = reinterpret_cast<f32x4*>(nsm);             // [NCH * 2][64]
  u32x4* s_w = reinterpret_cast<u32x4*>(nsm + NCH * 2048);  // [EP / 4][NCH * 4][64]
  int* s_cnt = reinterpret_cast<int*>(nsm + NCH * 2048 + EP * NCH * 1024);
  float(*s_p)[EP] = reinterpret_cast<float(*)[EP]>(s_cnt + EP);  // [NWV][EP]
  float* s_z = reinterpret_cast<float*>(s_p + NWV);              // [NWV]
  int* s_nf = reinterpret_cast<int*>(s_z + NWV);                 // [NWV]
  int* s_last = s_nf + NWV;
  float* s_fin = reinterpret_cast<float*>(s_last + 4);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = norm_wave();
  const int N = a.N, H = a.H, E = a.E, K = a.K;
  const uint16_t* __restrict__ x = static_cast<const uint16_t*>(a.x);
  uint16_t* __restrict__ xn = static_cast<uint16_t*>(a.xn);
  const int rowbytes = H * 2;
  const int nwt = gridDim.x * NWV;
  auto rows = [&](int t) { return buf_rsrc(x + (int64_t)t * H, t < N ? rowbytes : 0); };
  int t0 = blockIdx.x * NWV + wv;
  RowFrag<uint16_t, NCH> f[R];  // the first rows are requested before the LDS staging (their latencies overlap)
  if (t0 < N) {
#pragma unroll
    for (int r = 0; r < R; ++r) frag_load_all(f[r], rows(t0 + r * nwt), lane);
  }
  stage_gamma<TG, NCH>(s_gam, static_cast<const TG*>(a.gamma), H, tid, NT);
  stage_gate_fwd<NCH, EP>(s_w, a.wg, H, E, tid, NT);
  if (tid < EP) s_cnt[tid] = 0;
  __syncthreads();

  const int el = lane & 15;                           // expert of this lane inside its 16-lane row
  const int tr = R == 2 ? lane >> 5 : 0;              // token this lane routes
  const bool lead = (lane & (R == 2 ? 16 : 48)) == 0;  // the 16-lane row whose results are stored
  const bool real = el < E;
  const bool has_bias = a.bias != nullptr;
  const float bias_v = (has_bias && real) ? a.bias[el] : 0.f;
  float pacc = 0.f, zacc = 0.f;
  int nfacc = 0;

  for (; t0 < N; t0 += R * nwt) {
    row_fence();
    buf_rsrc_t rn[R];
    float rs[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int tr_ = t0 + r * nwt;
      rn[r] = rows(tr_ + R * nwt);
      rs[r] = rsqrtf(frag_sumsq(f[r]) / (float)H + a.eps);
      if (lane == 0 && tr_ < N) a.rstd[tr_] = rs[r];
    }
    float acc[NV];
#pragma unroll
    for (int e = 0; e < NV; ++e) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float v[8], g[8], o[8];
      u32x4 pk[R];
      const int c = lane + 64 * j;
      gamma_get<NCH>(s_gam, j, lane, g);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int tr_ = t0 + r * nwt;
        frag_get(f[r], j, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = (v[i] * rs[r]) * g[i];
        chunk_store<uint16_t>(xn + (int64_t)tr_ * H, c, tr_ < N && 8 * c < H, o, pk[r]);
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int q = 0; q < EP / 4; ++q) {
          const u32x4 wq = s_w[((q * NCH + j) * 4 + m) * 64 + lane];
#pragma unroll
          for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r * EP + 4 * q + k] = dot2bf(pk[r][m], wq[k], acc[r * EP + 4 * q + k]);
        }
#pragma unroll
      for (int r = 0; r < R; ++r) frag_load(f[r], rn[r], j, lane);  // the next rows' chunk j into the freed registers
      chunk_fence(acc);
    }
    // ---- logits: the wave total of (token, expert) i ends in lanes i * (64 / NV) ..; gather token tr's
    // expert el to lane el of the token's 16-lane rows ----
    const float tot = wave_reduce_scatter<NV>(acc, lane);
    float lg = __shfl(tot, (tr * EP + (el < EP ? el : 0)) * (64 / NV));
    const int t = t0 + tr * nwt;
    const bool vt = t < N;
    if (has_bias) lg += bias_v;
    if (lead && real && vt) a.logits[(int64_t)t * E + el] = lg;
    nfacc += __popcll(__ballot(lead && real && vt && !isfinite(lg)));
    const float rv = (!real || lg != lg) ? -INFINITY : lg;  // NaN never wins a top-k slot
    const float m = row16_max(rv);
    const float ex = real ? expf(rv - m) : 0.f;
    const float s = row16_sum(ex);
    const float inv = 1.f / s;
    const float lse = m + logf(s);
    if (lead && el == 0 && vt) a.lse[t] = lse;
    zacc += vt ? lse * lse : 0.f;
    pacc += vt ? ex * inv : 0.f;
    // top-k: K rounds of arg-max (larger logit, lower id on a tie) over the experts not taken yet
    uint32_t key = real ? order_key(rv) : 0u;
    int my_e = 0;
    float my_p = 0.f, psum = 0.f;
    for (int rk = 0; rk < K; ++rk) {
      uint32_t bk = key;
      int be = el;
      row16_argmax_key(bk, be);
      const float pv = expf(order_val(bk) - m) * inv;
      psum += pv;
      key = el == be ? 0u : key;
      my_e = el == rk ? be : my_e;
      my_p = el == rk ? pv : my_p;
    }
    const float rden = 1.f / fmaxf(psum, 1e-30f);
    if (lead && el < K && vt) {
      a.idx[(int64_t)t * K + el] = my_e;
      store_f(a.w, a.w_dt, (int64_t)t * K + el, my_p * rden);
      atomicAdd(&s_cnt[my_e], 1);
    }
  }
  if constexpr (R == 2) {  // the two tokens' accumulators (lanes l and l + 32) in a fixed order
    pacc += __shfl_xor(pacc, 32);
    zacc += __shfl_xor(zacc, 32);
  }
  if (lane < EP) s_p[wv][lane] = pacc;
  if (lane == 0) {
    s_z[wv] = zacc;
    s_nf[wv] = nfacc;
  }
  __syncthreads();
  // ---- block partials (waves summed in order), then the last block folds all of them ----
  if (tid < E) {
    float p = s_p[0][tid];
#pragma unroll
    for (int w = 1; w < NWV; ++w) p += s_p[w][tid];
    st_part(&a.part_cnt[(int64_t)blockIdx.x * E + tid], s_cnt[tid]);
    st_part(&a.part_p[(int64_t)blockIdx.x * E + tid], p);
  }
  if (tid == 0) {
    float zs = s_z[0];
    int nf = s_nf[0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) {
      zs += s_z[w];
      nf += s_nf[w];
    }
    st_part(&a.part_z[2 * blockIdx.x], zs);
    st_part(&a.part_z[2 * blockIdx.x + 1], (float)nf);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    *s_last = __hip_atomic_fetch_add(a.ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!*s_last) return;
  router_finalize_block<NT, true>(a.part_cnt, a.part_p, a.part_z, gridDim.x, N, E, K, a.aux_coef, a.z_coef, a.cnt,
                                  a.stats, a.aux, a.z, s_fin);
  if (tid == 0) *a.ticket = 0u;
}

// ---------------------------------------------------------------------------
// Backward.
// ---------------------------------------------------------------------------
struct NormBwdArgs {
  const void* x;
  const void* gamma;
  const float* rstd;
  const void* dxn;    // may be null (no gradient of xn from the expert path)
  const void* dxn2;   // MODE 1: a second gradient of xn
  const uint16_t* G;  // MODE 8 / 16: dL/dlogits, bf16 [N][MODE]
  const uint16_t* wg;  // MODE 8 / 16: gate [H, E] bf16
  int E;
  int N, H;
  void* dx;
  float* part_dg;  // [gridDim.x][H]
};

// MODE: 0 = dxn, 1 = dxn + dxn2, 8 / 16 = dxn + G wg^T with E <= MODE experts.
template <int NCH, int MODE>
constexpr size_t norm_bwd_lds() { return (size_t)NCH * 4096 + (MODE >= 8 ? (size_t)MODE * NCH * 1024 : 0); }

// Two waves per SIMD up to H = 4096 (the row state takes about 256 VGPRs there); wider rows take one.  With
// the gate image in LDS (MODE 8 / 16) one block fills a CU's LDS, so those blocks have eight waves.
template <int MODE>
constexpr int norm_bwd_waves() { return MODE >= 8 ? 8 : 4; }

template <typename TX, typename TG, int NCH, int MODE>
__global__ __launch_bounds__(norm_bwd_waves<MODE>() * 64) __attribute__((amdgpu_waves_per_eu(NCH <= 8 ? 2 : 1)))
void k_rmsnorm_bwd(NormBwdArgs a) {
  constexpr bool TWO = MODE == 1;
  constexpr int EP = MODE >= 8 ? MODE : 0;
  constexpr int NWV = norm_bwd_waves<MODE>();
  constexpr int NT = NWV * 64;
  extern __shared__ __attribute__((aligned(16))) uint8_t nsm[];
  f32x4* s_gam = reinterpret_cast<f32x4*>(nsm);             // [NCH * 2][64]
  f32x4* s_dg = s_gam + NCH * 128;                           // [NCH * 2][64]
  u32x4* s_w = reinterpret_cast<u32x4*>(s_dg + NCH * 128);  // [EP / 8][NCH * 8][64]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = norm_wave();
  const int N = a.N, H = a.H;
  const TX* __restrict__ x = static_cast<const TX*>(a.x);
  const TX* __restrict__ dxn = static_cast<const TX*>(a.dxn);
  const TX* __restrict__ dxn2 = static_cast<const TX*>(a.dxn2);
  TX* __restrict__ dx = static_cast<TX*>(a.dx);
  const int rowbytes = H * (int)sizeof(TX);
  const int nwt = gridDim.x * NWV;
  int t = blockIdx.x * NWV + wv;
  // a null gradient (or a row past N) reads as zeros through a descriptor with no records
  auto rows = [&](const TX* base, int row) {
    return buf_rsrc(base ? base + (int64_t)row * H : x, (base && row < N) ? rowbytes : 0);
  };
  RowFrag<TX, NCH> fx, fg, fg2;  // the first row is requested before the LDS staging (latencies overlap)
  if (t < N) {
    frag_load_all(fx, rows(x, t), lane);
    frag_load_all(fg, rows(dxn, t), lane);
    if constexpr (TWO) frag_load_all(fg2, rows(dxn2, t), lane);
  }
  stage_gamma<TG, NCH>(s_gam, static_cast<const TG*>(a.gamma), H, tid, NT);
  if constexpr (EP > 0)
    stage_gate_bwd<NCH, EP>(s_w, a.wg, H, a.E, tid, NT);
  __syncthreads();

  float dg[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) dg[j][i] = 0.f;
  for (; t < N; t += nwt) {
    row_fence();
    const int tn = t + nwt;
    const buf_rsrc_t rx = rows(x, tn), rg = rows(dxn, tn), rg2 = rows(TWO ? dxn2 : nullptr, tn);
    const float r = a.rstd[t];
    u32x4 gt[EP >= 8 ? EP / 8 : 1];
    if constexpr (EP > 0) {
#pragma unroll
      for (int q = 0; q < EP / 8; ++q) gt[q] = *reinterpret_cast<const u32x4*>(a.G + (int64_t)t * EP + 8 * q);
    }
    // pass 1: u = dxn (+ dxn2 | + G wg^T), rounded to the storage type as a sum of gradients of xn is;
    // c = sum_h gamma u xhat; dgamma += u xhat
    RowFrag<TX, NCH> fu;
    float c = 0.f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float v[8], gd[8], gm[8];
      frag_get(fx, j, v);
      frag_get(fg, j, gd);
      if constexpr (TWO) {
        float g2[8];
        frag_get(fg2, j, g2);
#pragma unroll
        for (int i = 0; i < 8; ++i) gd[i] += g2[i];
      }
      if constexpr (EP > 0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float d = 0.f;
#pragma unroll
          for (int q = 0; q < EP / 8; ++q) {
            const u32x4 wq = s_w[((q * NCH + j) * 8 + i) * 64 + lane];
#pragma unroll
            for (int m = 0; m < 4; ++m) d = dot2bf(wq[m], gt[q][m], d);
          }
          gd[i] += d;
        }
      }
      if constexpr (std::is_same<TX, uint16_t>::value) {
#pragma unroll
        for (int m = 0; m < 4; ++m) fu.w[j][m] = pack2bf(gd[2 * m], gd[2 * m + 1]);
      } else {
        fu.w[2 * j] = u32x4{__float_as_uint(gd[0]), __float_as_uint(gd[1]), __float_as_uint(gd[2]),
                            __float_as_uint(gd[3])};
        fu.w[2 * j + 1] = u32x4{__float_as_uint(gd[4]), __float_as_uint(gd[5]), __float_as_uint(gd[6]),
                                __float_as_uint(gd[7])};
      }
      frag_get(fu, j, gd);
      gamma_get<NCH>(s_gam, j, lane, gm);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float xh = v[i] * r;
        c = fmaf(gm[i] * gd[i], xh, c);
        dg[j][i] = fmaf(gd[i], xh, dg[j][i]);
      }
      frag_load(fg, rg, j, lane);
      if constexpr (TWO) frag_load(fg2, rg2, j, lane);
      chunk_fence(dg[j]);
      __asm__ volatile("" : "+v"(c));
    }
    c = wave_total(c) / (float)H;
    // pass 2: dx = r (gamma u - xhat c)
    TX* drow = dx + (int64_t)t * H;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      float v[8], gm[8], o[8], uu[8];
      frag_get(fx, j, v);
      frag_get(fu, j, uu);
      gamma_get<NCH>(s_gam, j, lane, gm);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = r * (gm[i] * uu[i] - (v[i] * r) * c);
      const int cc = lane + 64 * j;
      u32x4 pk;
      chunk_store<TX>(drow, cc, 8 * cc < H, o, pk);
      frag_load(fx, rx, j, lane);
      chunk_fence();
    }
  }
  // dgamma: the block's waves summed in order in LDS, one partial row per block
#pragma unroll
  for (int w = 0; w < NWV; ++w) {
    if (wv == w) {
#pragma unroll
      for (int j = 0; j < NCH; ++j)
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int k = (2 * j + q) * 64 + lane;
          const f32x4 d = {dg[j][4 * q], dg[j][4 * q + 1], dg[j][4 * q + 2], dg[j][4 * q + 3]};
          s_dg[k] = w == 0 ? d : s_dg[k] + d;
        }
    }
    __syncthreads();
  }
  for (int i = tid; i < NCH * 128; i += NT) {
    const int l = i & 63, q = (i >> 6) & 1, j = i >> 7;
    const int h0 = 8 * (l + 64 * j) + 4 * q;
    if (h0 < H) *reinterpret_cast<f32x4*>(a.part_dg + (int64_t)blockIdx.x * H + h0) = s_dg[i];
  }
}

// dgamma[h] = sum over blocks b of part_dg[b][h] in a fixed order.  Block = 32 columns x 32 groups of
// blocks: thread (g, cq) sums blocks g, g + 32, ... of columns 4 cq .. 4 cq + 3 (16-byte loads, four in
// flight), then the group sums are added in group order.
__global__ __launch_bounds__(256) void k_rmsnorm_dgamma(const float* __restrict__ part_dg, int nblk, int H,
                                                       void* __restrict__ dgamma, int g_dt) {
  __shared__ f32x4 s_acc[32][8];
  const int cq = threadIdx.x & 7, g = threadIdx.x >> 3;
  const int h0 = blockIdx.x * 32 + 4 * cq;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (h0 < H) {  // H % 8 == 0: the four columns are in range
    int b = g;
    for (; b + 96 < nblk; b += 128) {
      f32x4 v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = *reinterpret_cast<const f32x4*>(part_dg + (int64_t)(b + 32 * u) * H + h0);
#pragma unroll
      for (int u = 0; u < 4; ++u) acc += v[u];
    }
    for (; b < nblk; b += 32) acc += *reinterpret_cast<const f32x4*>(part_dg + (int64_t)b * H + h0);
  }
  s_acc[g][cq] = acc;
  __syncthreads();
  if (g == 0 && h0 < H) {
    f32x4 t = s_acc[0][cq];
#pragma unroll
    for (int gg = 1; gg < 32; ++gg) t += s_acc[gg][cq];
#pragma unroll
    for (int k = 0; k < 4; ++k) store_f(dgamma, g_dt, h0 + k, t[k]);
  }
}

namespace {

int norm_nch(int64_t H) { return H <= 512 ? 1 : H <= 2048 ? 4 : H <= 4096 ? 8 : 16; }
int norm_fwd_blocks(int64_t N) { return (int)std::min<int64_t>(1024, std::max<int64_t>(1, (N + 3) / 4)); }
// one block of eight waves per CU; one partial set per block for the statistics fold
constexpr int kRouteRows = 1;  // one row per wave, 16 waves a block (slightly ahead of two rows, 8 waves)
int norm_route_blocks(int64_t N) {
  constexpr int nw = route_waves<kRouteRows>() * kRouteRows;
  return (int)std::min<int64_t>(256, std::max<int64_t>(1, (N + nw - 1) / nw));
}
// the backward writes one dgamma partial row per block: about two blocks per CU
int norm_bwd_blocks(int64_t N) { return (int)std::min<int64_t>(512, std::max<int64_t>(1, (N + 3) / 4)); }
// the fused backward: one block of eight waves per CU
int norm_route_bwd_blocks(int64_t N) { return (int)std::min<int64_t>(256, std::max<int64_t>(1, (N + 7) / 8)); }
int norm_route_ep(int64_t E) { return E <= 8 ? 8 : 16; }
size_t align256n(size_t v) { return (v + 255) & ~(size_t)255; }

#define MOE_NCH(nch, CALL)                                  \
  do {                                                      \
    if (nch == 1) { constexpr int NCHv = 1; CALL; }         \
    else if (nch == 4) { constexpr int NCHv = 4; CALL; }    \
    else if (nch == 8) { constexpr int NCHv = 8; CALL; }    \
    else { constexpr int NCHv = 16; CALL; }                 \
  } while (0)

#define MOE_NORM_DT(xdt, gdt, CALL)                                                             \
  do {                                                                                          \
    if (xdt == MOE_BF16 && gdt == MOE_F32) { using TX = uint16_t; using TG = float; CALL; }     \
    else if (xdt == MOE_BF16) { using TX = uint16_t; using TG = uint16_t; CALL; }               \
    else if (gdt == MOE_F32) { using TX = float; using TG = float; CALL; }                      \
    else { using TX = float; using TG = uint16_t; CALL; }                                       \
  } while (0)

size_t route_lds(int nch, int ep) {
  size_t b = 0;
  MOE_NCH(nch, b = (ep == 8 ? norm_route_lds<NCHv, 8, kRouteRows>() : norm_route_lds<NCHv, 16, kRouteRows>()));
  return b;
}
size_t route_bwd_lds(int nch, int ep) {
  size_t b = 0;
  MOE_NCH(nch, b = (ep == 8 ? norm_bwd_lds<NCHv, 8>() : norm_bwd_lds<NCHv, 16>()));
  return b;
}
constexpr size_t kNormLdsMax = 160 * 1024;
// the fused kernels take bf16 x and gate with E <= 16, and the gate image must fit in LDS
bool norm_route_fits(int64_t H, int64_t E) {
  return E <= 16 && route_lds(norm_nch(H), norm_route_ep(E)) <= kNormLdsMax;
}
bool norm_route_bwd_fits(int64_t H, int64_t E) {
  return router_dw_g_applies(H, E) && route_bwd_lds(norm_nch(H), norm_route_ep(E)) <= kNormLdsMax;
}

// Dynamic LDS above the default limit needs the kernel's attribute raised once.
template <typename K>
int allow_lds(K kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return check_launch("hipFuncSetAttribute");
  return 0;
}

bool al16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int norm_check(const char* what, int64_t N, int64_t H, int x_dt, int g_dt) {
  if (N < 0 || H < 8 || H % 8 || H > kNormMaxH)
    return fail_arg("%s: bad shape N=%lld H=%lld (need H %% 8 == 0, 8 <= H <= %d)", what, (long long)N, (long long)H,
                    kNormMaxH);
  if (N > INT32_MAX / 2) return fail_arg("%s: N too large", what);
  if ((x_dt != MOE_F32 && x_dt != MOE_BF16) || (g_dt != MOE_F32 && g_dt != MOE_BF16))
    return fail_arg("%s: unsupported dtype", what);
  return 0;
}

template <typename TX, typename TG, int NCH>
int launch_norm_fwd(int nblk, hipStream_t s, const NormFwdArgs& a) {
  constexpr size_t lds = norm_fwd_lds<NCH>();
  if (int rc = allow_lds(k_rmsnorm_fwd<TX, TG, NCH>, lds)) return rc;
  MOE_LAUNCH("k_rmsnorm_fwd", (k_rmsnorm_fwd<TX, TG, NCH>), dim3(nblk), dim3(256), lds, s, a);
  return check_launch("k_rmsnorm_fwd");
}

template <typename TG, int NCH, int EP>
int launch_norm_route(int nblk, hipStream_t s, const NormFwdArgs& a) {
  constexpr size_t lds = norm_route_lds<NCH, EP, kRouteRows>();
  if (int rc = allow_lds(k_rmsnorm_route<TG, NCH, EP, kRouteRows>, lds)) return rc;
  MOE_LAUNCH("k_rmsnorm_route", (k_rmsnorm_route<TG, NCH, EP, kRouteRows>), dim3(nblk),
             dim3(route_waves<kRouteRows>() * 64), lds, s, a);
  return check_launch("k_rmsnorm_route");
}

template <typename TX, typename TG, int NCH, int MODE>
int launch_norm_bwd(int nblk, hipStream_t s, const NormBwdArgs& a) {
  constexpr size_t lds = norm_bwd_lds<NCH, MODE>();
  constexpr const char* name = MODE >= 8 ? "k_rmsnorm_route_bwd" : "k_rmsnorm_bwd";
  if (int rc = allow_lds(k_rmsnorm_bwd<TX, TG, NCH, MODE>, lds)) return rc;
  MOE_LAUNCH(name, (k_rmsnorm_bwd<TX, TG, NCH, MODE>), dim3(nblk), dim3(norm_bwd_waves<MODE>() * 64), lds, s, a);
  return check_launch(name);
}

int launch_dgamma(hipStream_t s, const float* part, int nblk, int64_t H, void* dgamma, int g_dt) {
  MOE_LAUNCH("k_rmsnorm_dgamma", k_rmsnorm_dgamma, dim3((unsigned)((H + 31) / 32)), dim3(256), 0, s, part, nblk,
             (int)H, dgamma, g_dt);
  return check_launch("k_rmsnorm_dgamma");
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
  NormFwdArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  a.N = (int)N;
  a.H = (int)H;
  a.xn = xn_out;
  a.rstd = rstd_out;
  const int nblk = norm_fwd_blocks(N);
  int rc = 0;
  MOE_NORM_DT(x_dtype, gamma_dtype, MOE_NCH(norm_nch(H), rc = (launch_norm_fwd<TX, TG, NCHv>(nblk, s, a))));
  return rc;
}

extern "C" size_t moe_rmsnorm_router_fwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype,
                                                   int wg_dtype) {
  if (N <= 0 || H <= 0 || E <= 0) return 0;
  const int nblk = norm_route_blocks(N);
  const size_t fused = 256 + 2 * align256n((size_t)nblk * E * 4) + align256n((size_t)nblk * 2 * 4);
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
                     al16p(gamma) && al16p(xn_out) && al16p(wg) && (w_dtype == MOE_F32 || w_dtype == MOE_BF16);
  if (!fused) {
    // the norm, then the router over its output (the streaming / MFMA router kernels)
    if (int rc = moe_rmsnorm_fwd(x, x_dtype, gamma, gamma_dtype, eps, N, H, xn_out, rstd_out, stream)) return rc;
    return moe_router_fwd(xn_out, x_dtype, wg, wg_dtype, bias, N, H, E, K, idx_out, w_out, w_dtype, logits_out,
                          lse_out, cnt_out, stats_out, aux_coef, z_coef, aux_out, z_out, workspace, ws_bytes, stream);
  }
  if (!wg || !idx_out || !w_out || !logits_out || !lse_out || !cnt_out || !stats_out || !rstd_out)
    return fail_arg("moe_rmsnorm_router_fwd: null pointer argument");
  const int nblk = norm_route_blocks(N);
  const int nch = norm_nch(H), ep = norm_route_ep(E);
  const size_t off_cnt = 256, off_p = off_cnt + align256n((size_t)nblk * E * 4),
               off_z = off_p + align256n((size_t)nblk * E * 4), total = off_z + align256n((size_t)nblk * 2 * 4);
  if (ws_bytes < total || !workspace)
    return set_error("moe_rmsnorm_router_fwd: workspace %zu < %zu bytes", ws_bytes, total), MOE_EWORKSPACE;
  // the completion counter is the first word of the workspace: zero on entry, left zero (as the router's)
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  NormFwdArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.eps = eps;
  a.N = (int)N;
  a.H = (int)H;
  a.xn = xn_out;
  a.rstd = rstd_out;
  a.wg = static_cast<const uint16_t*>(wg);
  a.bias = bias;
  a.E = (int)E;
  a.K = (int)K;
  a.idx = idx_out;
  a.w = w_out;
  a.w_dt = w_dtype;
  a.logits = logits_out;
  a.lse = lse_out;
  a.part_cnt = reinterpret_cast<int*>(ws + off_cnt);
  a.part_p = reinterpret_cast<float*>(ws + off_p);
  a.part_z = reinterpret_cast<float*>(ws + off_z);
  a.ticket = reinterpret_cast<unsigned*>(ws);
  a.aux_coef = aux_coef;
  a.z_coef = z_coef;
  a.cnt = cnt_out;
  a.stats = stats_out;
  a.aux = aux_out;
  a.z = z_out;
  int rc = 0;
  if (gamma_dtype == MOE_F32)
    MOE_NCH(nch, rc = (ep == 8 ? launch_norm_route<float, NCHv, 8>(nblk, s, a)
                               : launch_norm_route<float, NCHv, 16>(nblk, s, a)));
  else
    MOE_NCH(nch, rc = (ep == 8 ? launch_norm_route<uint16_t, NCHv, 8>(nblk, s, a)
                               : launch_norm_route<uint16_t, NCHv, 16>(nblk, s, a)));
  return rc;
}

extern "C" size_t moe_rmsnorm_bwd_workspace(int64_t N, int64_t H) {
  if (N <= 0 || H <= 0) return 0;
  return align256n((size_t)norm_bwd_blocks(N) * H * 4);
}

extern "C" int moe_rmsnorm_bwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, const float* rstd,
                               const void* dxn, const void* dxn2, int64_t N, int64_t H, void* dx_out,
                               void* dgamma_out, void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = norm_check("moe_rmsnorm_bwd", N, H, x_dtype, gamma_dtype)) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (!gamma || !dgamma_out) return fail_arg("moe_rmsnorm_bwd: null pointer argument");
  if (N == 0) return launch_dgamma(s, nullptr, 0, H, dgamma_out, gamma_dtype);
  if (!x || !rstd || !dxn || !dx_out || !al16p(x) || !al16p(gamma) || !al16p(dxn) || !al16p(dx_out) ||
      (dxn2 && !al16p(dxn2)))
    return fail_arg("moe_rmsnorm_bwd: null or misaligned pointer");
  const int nblk = norm_bwd_blocks(N);
  if (ws_bytes < moe_rmsnorm_bwd_workspace(N, H) || !workspace)
    return set_error("moe_rmsnorm_bwd: workspace too small"), MOE_EWORKSPACE;
  float* part = static_cast<float*>(workspace);
  NormBwdArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.rstd = rstd;
  a.dxn = dxn;
  a.dxn2 = dxn2;
  a.N = (int)N;
  a.H = (int)H;
  a.dx = dx_out;
  a.part_dg = part;
  int rc = 0;
  if (dxn2)
    MOE_NORM_DT(x_dtype, gamma_dtype, MOE_NCH(norm_nch(H), rc = (launch_norm_bwd<TX, TG, NCHv, 1>(nblk, s, a))));
  else
    MOE_NORM_DT(x_dtype, gamma_dtype, MOE_NCH(norm_nch(H), rc = (launch_norm_bwd<TX, TG, NCHv, 0>(nblk, s, a))));
  if (rc) return rc;
  return launch_dgamma(s, part, nblk, H, dgamma_out, gamma_dtype);
}

namespace {
// workspace layout of the fused backward: G, the router's dwg partials, the gate image, the dgamma partials
struct NormRouteBwdPlan {
  bool fused;
  int nch, ep, nblk;
  size_t off_g, off_rw, off_dg, total;
};
NormRouteBwdPlan plan_norm_route_bwd(int64_t N, int64_t H, int64_t E, int64_t K, int x_dt, int wg_dt) {
  NormRouteBwdPlan p{};
  p.fused = x_dt == MOE_BF16 && wg_dt == MOE_BF16 && norm_route_bwd_fits(H, E);
  p.nch = norm_nch(H);
  p.ep = norm_route_ep(E);
  p.nblk = p.fused ? norm_route_bwd_blocks(N) : norm_bwd_blocks(N);
  if (p.fused) {
    p.off_g = 0;
    p.off_rw = align256n((size_t)N * p.ep * 2);
    p.off_dg = p.off_rw + router_dw_g_workspace(N, H, E);
    p.total = p.off_dg + moe_rmsnorm_bwd_workspace(N, H);
  } else {
    // the router backward writes its dxn into the workspace; the norm backward adds it to the caller's
    const size_t esz = x_dt == MOE_BF16 ? 2 : 4;
    p.off_g = 0;
    p.off_rw = align256n((size_t)N * H * esz);
    p.off_dg = p.off_rw + moe_router_bwd_workspace(N, H, E, K, x_dt, wg_dt);
    p.total = p.off_dg + moe_rmsnorm_bwd_workspace(N, H);
  }
  return p;
}
}  // namespace

extern "C" size_t moe_rmsnorm_router_bwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype,
                                                   int wg_dtype) {
  if (N <= 0 || H <= 0 || E <= 0) return 0;
  return plan_norm_route_bwd(N, H, E, K, x_dtype, wg_dtype).total;
}

extern "C" int moe_rmsnorm_router_bwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype,
                                      const float* rstd, const void* xn, const void* wg, int wg_dtype,
                                      const float* logits, const int64_t* idx, const void* grad_w, int gw_dtype,
                                      const int64_t* cnt, const float* grad_aux, const float* grad_z, float aux_coef,
                                      float z_coef, const void* dxn, int64_t N, int64_t H, int64_t E, int64_t K,
                                      void* dx_out, void* dgamma_out, void* dwg_out, void* workspace, size_t ws_bytes,
                                      void* stream) {
  if (int rc = norm_check("moe_rmsnorm_router_bwd", N, H, x_dtype, gamma_dtype)) return rc;
  if (E < 1 || E > kMaxE || K < 1 || K > E)
    return fail_arg("moe_rmsnorm_router_bwd: bad shape E=%lld K=%lld", (long long)E, (long long)K);
  if ((wg_dtype != MOE_F32 && wg_dtype != MOE_BF16) || (gw_dtype != MOE_F32 && gw_dtype != MOE_BF16))
    return fail_arg("moe_rmsnorm_router_bwd: unsupported dtype");
  if (!gamma || !dgamma_out || !wg || !dwg_out) return fail_arg("moe_rmsnorm_router_bwd: null pointer argument");
  if (aux_coef != 0.f && !cnt) return fail_arg("moe_rmsnorm_router_bwd: aux_coef != 0 needs cnt");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (N == 0) {
    if (int rc = launch_dgamma(s, nullptr, 0, H, dgamma_out, gamma_dtype)) return rc;
    return moe_router_bwd(xn ? xn : gamma, x_dtype, wg, wg_dtype, logits, idx, grad_w, gw_dtype, cnt, grad_aux,
                          grad_z, aux_coef, z_coef, 0, H, E, K, dx_out ? dx_out : dgamma_out, dwg_out, workspace,
                          ws_bytes, stream);
  }
  if (!x || !rstd || !xn || !logits || !idx || !dx_out || !al16p(x) || !al16p(gamma) || !al16p(xn) ||
      !al16p(dx_out) || (dxn && !al16p(dxn)))
    return fail_arg("moe_rmsnorm_router_bwd: null or misaligned pointer");
  const NormRouteBwdPlan p = plan_norm_route_bwd(N, H, E, K, x_dtype, wg_dtype);
  if (ws_bytes < p.total || !workspace)
    return set_error("moe_rmsnorm_router_bwd: workspace %zu < %zu bytes", ws_bytes, p.total), MOE_EWORKSPACE;
  char* ws = static_cast<char*>(workspace);
  float* part = reinterpret_cast<float*>(ws + p.off_dg);
  if (!p.fused) {
    // the router backward over xn (its dxn into the workspace), then the norm backward of dxn + that
    void* dxr = ws + p.off_g;
    if (int rc = moe_router_bwd(xn, x_dtype, wg, wg_dtype, logits, idx, grad_w, gw_dtype, cnt, grad_aux, grad_z,
                                aux_coef, z_coef, N, H, E, K, dxr, dwg_out, ws + p.off_rw, p.off_dg - p.off_rw,
                                stream))
      return rc;
    return moe_rmsnorm_bwd(x, x_dtype, gamma, gamma_dtype, rstd, dxn ? dxn : dxr, dxn ? dxr : nullptr, N, H, dx_out,
                           dgamma_out, part, p.total - p.off_dg, stream);
  }
  uint16_t* G = reinterpret_cast<uint16_t*>(ws + p.off_g);
  if (int rc = router_dw_g(static_cast<const uint16_t*>(xn), static_cast<const uint16_t*>(wg), logits, idx, grad_w,
                           gw_dtype, cnt, grad_aux, grad_z, aux_coef, z_coef, N, H, E, K, dwg_out, G, p.ep,
                           ws + p.off_rw, s))
    return rc;
  NormBwdArgs a{};
  a.x = x;
  a.gamma = gamma;
  a.rstd = rstd;
  a.dxn = dxn;
  a.G = G;
  a.wg = static_cast<const uint16_t*>(wg);
  a.E = (int)E;
  a.N = (int)N;
  a.H = (int)H;
  a.dx = dx_out;
  a.part_dg = part;
  int rc = 0;
  if (gamma_dtype == MOE_F32)
    MOE_NCH(p.nch, rc = (p.ep == 8 ? launch_norm_bwd<uint16_t, float, NCHv, 8>(p.nblk, s, a)
                                   : launch_norm_bwd<uint16_t, float, NCHv, 16>(p.nblk, s, a)));
  else
    MOE_NCH(p.nch, rc = (p.ep == 8 ? launch_norm_bwd<uint16_t, uint16_t, NCHv, 8>(p.nblk, s, a)
                                   : launch_norm_bwd<uint16_t, uint16_t, NCHv, 16>(p.nblk, s, a)));
  if (rc) return rc;
  return launch_dgamma(s, part, p.nblk, H, dgamma_out, gamma_dtype);
}
