// Fused top-k router, forward and backward, for gfx950.
//
// Forward (bf16 tokens x bf16 gate): streaming kernels move the token rows
// (and the gate, raw or pre-packed into MFMA fragment order) through an LDS
// ring by LDS-DMA and accumulate fp32 logits with v_mfma_f32_16x16x32_bf16;
// softmax, top-k and renormalisation run on the accumulators in registers,
// one token per 16-lane row, with DPP reductions inside the row and a
// branch-free top-k.  Dispatch counts, mean probabilities and the z statistic
// are reduced per block and folded in a fixed order by the last block to
// finish (router_fin.h) -- deterministic, no float atomics, no extra launch.
// A packed-gate register-streaming kernel with a separate finalize covers
// the other bf16 shapes; fp32 / mixed dtypes take a VALU logits kernel plus a
// route-from-logits kernel with the same epilogue semantics.
//
// Backward: G = dL/dlogits per token (formed inside the streaming dx / dwg
// kernel for E <= 32, by its own kernel otherwise); dx = G wg^T and
// dwg = x^T G by MFMA kernels tiled over (token chunk, 256 hidden columns):
// the x tile is read once, staged in LDS, used for the dwg partial, and dx
// is written back through LDS with 16-byte stores.  dwg partials per token
// chunk are summed in a fixed order by a second kernel.
#include <cstdarg>
#include <mutex>

#include "common.h"
#include "router_fin.h"

namespace moe {


// ---------------------------------------------------------------------------
// Gate pack: wg [H, E] bf16 -> wp[c][nt][lane] (16 bytes each) with
// element j of lane l = wg[c*32 + (l/16)*8 + j][nt*16 + l%16], zero padded.
// ---------------------------------------------------------------------------
__global__ void k_pack_gate(const uint16_t* __restrict__ wg, int H, int E, int NT, i16x8* __restrict__ wp,
                            unsigned* __restrict__ ticket) {
  if (ticket != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *ticket = 0u;
  const int64_t total = (int64_t)((H + 31) / 32) * NT * 64;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(q & 63);
    const int64_t r = q >> 6;
    const int nt = (int)(r % NT);
    const int c = (int)(r / NT);
    const int e = nt * 16 + (lane & 15);
    const int k0 = c * 32 + (lane >> 4) * 8;
    i16x8 v;
    const int ee = min(e, E - 1);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int k = k0 + j;
      const short val = (short)wg[(int64_t)min(k, H - 1) * E + ee];  // clamped: always in bounds
      v[j] = (e < E && k < H) ? val : (short)0;
    }
    wp[q] = v;
  }
}

// Routing epilogue of one 16-token group: acc[nt][i] = logits[t0 + g*4 + i][nt*16 + n] (16x16 MFMA
// layout).  Adds the bias, writes logits / lse / top-k ids / renormalised weights, counts the picks in
// s_cnt (LDS atomics) and leaves the group's probability sums, z sum and non-finite count in
// s_p[0 .. NT*16), *s_z, *s_nf.
template <int NT>
__device__ __forceinline__ void route_group(const f32x4 (&acc)[NT], int t0, int lane, const float* __restrict__ bias,
                                            int N, int E, int K, int64_t* __restrict__ idx_out,
                                            void* __restrict__ w_out, int w_dt, float* __restrict__ logits_out,
                                            float* __restrict__ lse_out, int* s_cnt, float* s_p, float* s_z,
                                            int* s_nf) {
  const int g = lane >> 4;
  const int n = lane & 15;
  float pacc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) pacc[nt] = 0.f;
  float zacc = 0.f;
  int nf = 0;
  // the lane's bias values, loaded once (a wave-uniform branch on bias: no per-token load or wait)
  float bv[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) bv[nt] = 0.f;
  if (bias != nullptr) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bv[nt] = bias[min(nt * 16 + n, E - 1)];
  }
  // The row of 16 lanes g owns tokens t0 + 4g + i, i < 4; the four tokens are processed side by side
  // (independent dependency chains for the scheduler to interleave).
  float lg[4][NT], m[4], inv[4];
  uint32_t kh[4][NT];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tt = t0 + g * 4 + i;
    const bool valid = tt < N;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int e = nt * 16 + n;
      float v = acc[nt][i];
      if (bias != nullptr && e < E) v += bv[nt];
      if (valid && e < E) {
        logits_out[(int64_t)tt * E + e] = v;
        if (!isfinite(v)) ++nf;
      }
      if (v != v) v = -INFINITY;  // NaN never wins a top-k slot
      lg[i][nt] = (e < E) ? v : -INFINITY;
    }
    float mi = lg[i][0];
#pragma unroll
    for (int nt = 1; nt < NT; ++nt) mi = fmaxf(mi, lg[i][nt]);
    m[i] = row16_max(mi);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tt = t0 + g * 4 + i;
    float ex[NT];
    float s = 0.f;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      ex[nt] = expf(lg[i][nt] - m[i]);
      s += ex[nt];
    }
    s = row16_sum(s);
    inv[i] = 1.f / s;
    const float lse = m[i] + logf(s);
    if (tt < N) {
      if (n == 0) lse_out[tt] = lse;
      zacc += lse * lse;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) pacc[nt] += ex[nt] * inv[i];
    }
    // order-preserving keys of the logits (0: no candidate, an expert past E or one already taken)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) kh[i][nt] = (nt * 16 + n < E) ? order_key(lg[i][nt]) : 0u;
  }

  // top-k: K rounds of a row arg-max over the keys; the lowest expert id wins a tie.  Round r's winner
  // is kept by lane r % 16 and its key is cleared in the lane that holds it.  Branch-free: per round and
  // token, a max over the lane's NT keys and four DPP exchange steps across the row.
  int e_slot0[4], e_slot1[4];
  float p_slot0[4], p_slot1[4], psum[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    e_slot0[i] = e_slot1[i] = 0;
    p_slot0[i] = p_slot1[i] = psum[i] = 0.f;
  }
  for (int r = 0; r < K; ++r) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t bh = kh[i][0];
      int bnt = 0;
#pragma unroll
      for (int nt = 1; nt < NT; ++nt) {  // strict '>' keeps the lower tile (lower id) on a tie
        const bool t = kh[i][nt] > bh;
        bh = t ? kh[i][nt] : bh;
        bnt = t ? nt : bnt;
      }
      int be = bh ? bnt * 16 + n : 0x7fffffff;
      row16_argmax_key(bh, be);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) kh[i][nt] = (be == nt * 16 + n) ? 0u : kh[i][nt];  // the winner's lane
      const float pv = expf(order_val(bh) - m[i]) * inv[i];
      psum[i] += pv;
      e_slot0[i] = r == n ? be : e_slot0[i];
      p_slot0[i] = r == n ? pv : p_slot0[i];
      e_slot1[i] = r == n + 16 ? be : e_slot1[i];
      p_slot1[i] = r == n + 16 ? pv : p_slot1[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int tt = t0 + g * 4 + i;
    const float rden = 1.f / fmaxf(psum[i], 1e-30f);
    if (tt < N) {
      if (n < K) {
        idx_out[(int64_t)tt * K + n] = e_slot0[i];
        store_f(w_out, w_dt, (int64_t)tt * K + n, p_slot0[i] * rden);
        atomicAdd(&s_cnt[e_slot0[i]], 1);
      }
      if (n + 16 < K) {
        idx_out[(int64_t)tt * K + n + 16] = e_slot1[i];
        store_f(w_out, w_dt, (int64_t)tt * K + n + 16, p_slot1[i] * rden);
        atomicAdd(&s_cnt[e_slot1[i]], 1);
      }
    }
  }
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float v = pacc[nt];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (g == 0) s_p[nt * 16 + n] = v;
  }
  zacc += __shfl_xor(zacc, 16);
  zacc += __shfl_xor(zacc, 32);
  nf = wave_sum(nf);
  if (lane == 0) {
    *s_z = zacc;
    *s_nf = nf;
  }
}

// Routing of one 16-token group with four lanes per token (the wide forward, NT = 4 or 8 tiles of 16 experts).
// acc[nt][i] = logits[t0 + 4g + i][nt*16 + n] (16x16 MFMA layout, lane = 16g + n).  The bias, the logits / nf
// outputs and the NaN mapping happen in that layout (64-byte row segments); the cleaned logits then go through
// `tile` (the wave's own LDS, 16 rows of NT*16 + 4 floats: the padding puts the 16 rows of one column group in
// different bank groups) so that lane 4r + s holds the 4*NT logits of token t0 + r at experts 4j + s.  Softmax,
// top-k (K rounds of a strict arg-max over order-preserving keys: within a lane the lowest j wins a tie, across
// the quad the lowest expert id) and renormalisation run on those with 2-step quad reductions (DPP), where the
// 16-lane form needs 4 steps per round and handles 4 tokens per lane in turn.  Round r's pick is kept by lane
// s = r % 4 in slot r / 4.  The probabilities go back through the tile to be summed per expert over the group
// in the MFMA layout.  Outputs and statistics (s_cnt, s_p, s_z, s_nf) as route_group's.
template <int NT>
__device__ __forceinline__ void route_quad(const f32x4 (&acc)[NT], float* tile, int t0, int lane,
                                           const float* __restrict__ bias, int N, int E, int K,
                                           int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt,
                                           float* __restrict__ logits_out, float* __restrict__ lse_out, int* s_cnt,
                                           float* s_p, float* s_z, int* s_nf) {
  constexpr int L = 4 * NT;       // logits per lane
  constexpr int P = NT * 16 + 4;  // tile row pitch (floats)
  constexpr int KS = kMaxK / 4;   // pick slots per lane
  const int g = lane >> 4, n = lane & 15;
  int nf = 0;
  {
    float bv[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) bv[nt] = (bias != nullptr) ? bias[min(nt * 16 + n, E - 1)] : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tt = t0 + g * 4 + i;
      const bool valid = tt < N;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int e = nt * 16 + n;
        float v = acc[nt][i] + bv[nt];
        if (valid && e < E) {
          logits_out[(int64_t)tt * E + e] = v;
          if (!isfinite(v)) ++nf;
        }
        if (v != v || e >= E) v = -INFINITY;  // NaN (and experts past E) never win a top-k slot
        tile[(4 * g + i) * P + nt * 16 + n] = v;
      }
    }
  }
  __asm__ volatile("" ::: "memory");  // the wave's LDS accesses complete in order: the tile is written
  const int r = lane >> 2, s = lane & 3;
  const int tt = t0 + r;
  const bool valid = tt < N;
  float lg[L];
#pragma unroll
  for (int j = 0; j < L; ++j) lg[j] = tile[r * P + 4 * j + s];
  float m = lg[0];
#pragma unroll
  for (int j = 1; j < L; ++j) m = fmaxf(m, lg[j]);
  m = fmaxf(m, row16_partner<0>(m));
  m = fmaxf(m, row16_partner<1>(m));
  float ex[L], sum = 0.f;
#pragma unroll
  for (int j = 0; j < L; ++j) {
    ex[j] = expf(lg[j] - m);
    sum += ex[j];
  }
  sum += row16_partner<0>(sum);
  sum += row16_partner<1>(sum);
  const float inv = 1.f / sum;
  const float lse = m + logf(sum);
  if (valid && s == 0) lse_out[tt] = lse;
  uint32_t kh[L];
#pragma unroll
  for (int j = 0; j < L; ++j) kh[j] = (4 * j + s < E) ? order_key(lg[j]) : 0u;
  int e_slot[KS];
  float p_slot[KS];
#pragma unroll
  for (int q = 0; q < KS; ++q) {
    e_slot[q] = 0;
    p_slot[q] = 0.f;
  }
  float psum = 0.f;
  for (int rr = 0; rr < K; ++rr) {
    uint32_t bh = kh[0];
    int bj = 0;
#pragma unroll
    for (int j = 1; j < L; ++j) {  // strict '>' keeps the lower j (lower expert) on a tie
      const bool t = kh[j] > bh;
      bh = t ? kh[j] : bh;
      bj = t ? j : bj;
    }
    int be = bh ? 4 * bj + s : 0x7fffffff;
    const uint32_t w1 = max(bh, (uint32_t)row16_partner<0>((int)bh));
    const uint32_t wmax = max(w1, (uint32_t)row16_partner<1>((int)w1));
    be = bh == wmax ? be : 0x7fffffff;
    be = min(be, row16_partner<0>(be));
    be = min(be, row16_partner<1>(be));
#pragma unroll
    for (int j = 0; j < L; ++j) kh[j] = (4 * j + s == be) ? 0u : kh[j];  // the winner's lane
    const float pv = expf(order_val(wmax) - m) * inv;
    psum += pv;
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      e_slot[q] = rr == 4 * q + s ? be : e_slot[q];
      p_slot[q] = rr == 4 * q + s ? pv : p_slot[q];
    }
  }
  const float rden = 1.f / fmaxf(psum, 1e-30f);
  if (valid) {
#pragma unroll
    for (int q = 0; q < KS; ++q) {
      const int rr = 4 * q + s;
      if (rr < K) {
        idx_out[(int64_t)tt * K + rr] = e_slot[q];
        store_f(w_out, w_dt, (int64_t)tt * K + rr, p_slot[q] * rden);
        atomicAdd(&s_cnt[e_slot[q]], 1);
      }
    }
  }
  // the token's probabilities back through the tile, summed per expert over the group's 16 tokens
  __asm__ volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < L; ++j) tile[r * P + 4 * j + s] = valid ? ex[j] * inv : 0.f;
  __asm__ volatile("" ::: "memory");
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) v += tile[(4 * g + i) * P + nt * 16 + n];
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    if (g == 0) s_p[nt * 16 + n] = v;
  }
  float zacc = (valid && s == 0) ? lse * lse : 0.f;
  zacc += __shfl_xor(zacc, 1);
  zacc += __shfl_xor(zacc, 2);
  zacc += __shfl_xor(zacc, 4);
  zacc += __shfl_xor(zacc, 8);
  zacc += __shfl_xor(zacc, 16);
  zacc += __shfl_xor(zacc, 32);
  nf = wave_sum(nf);
  if (lane == 0) {
    *s_z = zacc;
    *s_nf = nf;
  }
}

// Routing of a block's 16*TG tokens with one lane per token (E <= EP, EP = 8 or 16), called by every thread of
// the 512-thread block.  The 8 waves' partial logit tiles (s_accf: wave w's TG 16x16 tiles in MFMA layout,
// TG*256 floats) are summed in wave order into s_lg [16*TG][17] (rows padded: the per-token reads below hit
// distinct banks); then wave 0 routes token t0 + lane from its logits in registers: bias, the logits / lse
// outputs, softmax, top-k (K rounds of a strict arg-max over order-preserving keys, scanned from expert 0 so the
// lowest expert wins a tie), renormalised weights; it leaves each token's probabilities in its s_lg row and its
// picks as a bit mask in s_pick [64].  The per-expert statistics are then spread over the waves (wave w takes
// experts w and w + 8): pick counts by ballots, probability sums by DPP row sums and the four rows in order.
// Results: s_cnt[e], s_p[0][e], s_z[0], s_nf[0] (zeros in s_p[q] / s_z[q] / s_nf[q], q > 0, which the block
// tail also adds).
template <int TG, int EP>
__device__ __forceinline__ void route_lanes(const float* s_accf, float* s_lg, int* s_pick, int t0,
                                            const float* __restrict__ bias, int N, int E, int K,
                                            int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt,
                                            float* __restrict__ logits_out, float* __restrict__ lse_out, int* s_cnt,
                                            float (*s_p)[16], float* s_z, int* s_nf) {
  constexpr int NV = TG * 256;
  for (int v = threadIdx.x; v < NV; v += 512) {
    float a = s_accf[v];
#pragma unroll
    for (int w = 1; w < 8; ++w) a += s_accf[w * NV + v];
    const int q = v >> 8, ln = (v >> 2) & 63, i = v & 3;
    s_lg[(16 * q + 4 * (ln >> 4) + i) * 17 + (ln & 15)] = a;
  }
  for (int i = threadIdx.x; i < TG * 16; i += 512) {
    if (i >= 16) s_p[i >> 4][i & 15] = 0.f;
    if (i > 0 && i < TG) {
      s_z[i] = 0.f;
      s_nf[i] = 0;
    }
  }
  lds_sync();
  const int lane = threadIdx.x & 63;
  const bool valid = lane < 16 * TG && t0 + lane < N;
  // a row of 16 lanes sums its values, then the four row sums are added in row order
  auto wave_total = [&](float v) __attribute__((always_inline)) {
    v = row16_sum(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  };
  if (threadIdx.x < 64) {
    const int tt = t0 + lane;
    float* const row = s_lg + min(lane, 16 * TG - 1) * 17;
    float lg[EP];
    int nf = 0;
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      float v = row[e];
      if (e < E) {
        if (bias != nullptr) v += bias[e];  // wave-uniform address: scalar loads
        nf += (valid && !isfinite(v)) ? 1 : 0;
      }
      lg[e] = v;
    }
    if (valid) {
      float* lrow = logits_out + (int64_t)tt * E;
      if ((E & 3) == 0 && (reinterpret_cast<uintptr_t>(logits_out) & 15u) == 0) {
#pragma unroll
        for (int e = 0; e < EP; e += 4)
          if (e < E) *reinterpret_cast<f32x4*>(lrow + e) = f32x4{lg[e], lg[e + 1], lg[e + 2], lg[e + 3]};
      } else {
#pragma unroll
        for (int e = 0; e < EP; ++e)
          if (e < E) lrow[e] = lg[e];
      }
    }
    float m = -INFINITY;
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      float v = lg[e];
      if (v != v || e >= E) v = -INFINITY;  // NaN never wins a top-k slot
      lg[e] = v;
      m = fmaxf(m, v);
    }
    float ex[EP], sum = 0.f;
#pragma unroll
    for (int e = 0; e < EP; ++e) {
      ex[e] = expf(lg[e] - m);
      sum += ex[e];
    }
    const float inv = 1.f / sum;
    const float lse = m + logf(sum);
    if (valid) lse_out[tt] = lse;
    uint32_t kh[EP];
#pragma unroll
    for (int e = 0; e < EP; ++e) kh[e] = e < E ? order_key(lg[e]) : 0u;
    // the K rounds run as a rolled loop (short code); a round's probability waits in the token's row
    uint32_t pick = 0u;
    float psum = 0.f;
#pragma unroll 1
    for (int r = 0; r < K; ++r) {
      uint32_t bh = 0u;
      int be = 0;
#pragma unroll
      for (int e = 0; e < EP; ++e) {
        const bool t = kh[e] > bh;
        bh = t ? kh[e] : bh;
        be = t ? e : be;
      }
#pragma unroll
      for (int e = 0; e < EP; ++e) kh[e] = e == be ? 0u : kh[e];
      const float pv = expf(order_val(bh) - m) * inv;
      psum += pv;
      pick |= 1u << be;
      if (valid) idx_out[(int64_t)tt * K + r] = be;
      if (lane < 16 * TG) row[r] = pv;
    }
    const float rden = 1.f / fmaxf(psum, 1e-30f);
    if (valid) {
#pragma unroll 1
      for (int r = 0; r < K; ++r) store_f(w_out, w_dt, (int64_t)tt * K + r, row[r] * rden);
    }
    if (lane < 16 * TG) {
#pragma unroll
      for (int e = 0; e < EP; ++e) row[e] = valid ? ex[e] * inv : 0.f;  // the token's probabilities
    }
    s_pick[lane] = valid ? (int)pick : 0;
    const float zs = wave_total(valid ? lse * lse : 0.f);
    const int nfs = __ballot(nf > 0) == 0ull ? 0 : wave_sum(nf);  // the reduction only when some lane has one
    if (lane == 0) {
      s_z[0] = zs;
      s_nf[0] = nfs;
    }
  }
  lds_sync();
  const int wv = threadIdx.x >> 6;
  const int pk = s_pick[lane];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int e = wv + 8 * h;
    const int c = (int)__popcll(__ballot((pk >> e) & 1));
    const float ps = e < E ? wave_total(lane < 16 * TG ? s_lg[lane * 17 + e] : 0.f) : 0.f;
    if (lane == 0) {
      if (e < E) s_cnt[e] = c;
      s_p[0][e] = ps;
    }
  }
}

// ---------------------------------------------------------------------------
// Forward, bf16 x bf16, MFMA.
//   NT: 16-expert tiles (ceil(E/16)).  HS: waves sharing one 16-token group,
//   each streaming 1/HS of the hidden dim (partial logits are summed in LDS
//   in a fixed order).  U: 32-wide k-chunks per prefetch group; the main
//   loop is branch-free and double-buffered (2U chunks in flight per wave).
// Block = 4 waves = 4/HS token groups of 16 tokens.
// ---------------------------------------------------------------------------
template <int NT, int HS, int U>
__global__ __launch_bounds__(256) void k_router_fwd_bf16(
    const uint16_t* __restrict__ x, const i16x8* __restrict__ wp, const float* __restrict__ bias, int N, int H,
    int E, int K, int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt, float* __restrict__ logits_out,
    float* __restrict__ lse_out, int* __restrict__ part_cnt, float* __restrict__ part_p, float* __restrict__ part_z) {
  constexpr int TG = 4 / HS;
  __shared__ int s_cnt[NT * 16];
  __shared__ float s_p[TG][NT * 16];
  __shared__ float s_z[TG];
  __shared__ int s_nf[TG];
  __shared__ f32x4 s_acc[HS > 1 ? (HS - 1) * TG * NT * 64 : 1];

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int tg = wv / HS;
  const int hp = wv % HS;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int t0 = blockIdx.x * (16 * TG) + tg * 16;

  for (int i = threadIdx.x; i < NT * 16; i += blockDim.x) s_cnt[i] = 0;

  int row = t0 + n;
  if (row > N - 1) row = N - 1;
  const i16x8* xa = reinterpret_cast<const i16x8*>(x + (int64_t)row * H) + g;
  const i16x8* wb = wp + lane;
  const int nc = H >> 5;
  const int per = nc / HS;
  const int c_beg = hp * per;
  const int c_end = (hp == HS - 1) ? nc : c_beg + per;

  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (t0 < N) {
    i16x8 a0[U], a1[U];
    i16x8 b0[U][NT], b1[U][NT];
    auto load_grp = [&](i16x8(&a)[U], i16x8(&b)[U][NT], int c) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        a[u] = __builtin_nontemporal_load(xa + (c + u) * 4);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) b[u][nt] = wb[((c + u) * NT + nt) * 64];
      }
    };
    auto mma_grp = [&](const i16x8(&a)[U], const i16x8(&b)[U][NT]) {
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[nt] = mfma16x16x32(__builtin_bit_cast(bf16x8, a[u]), __builtin_bit_cast(bf16x8, b[u][nt]), acc[nt]);
    };
    int c = c_beg;
    const int npair = (c_end - c_beg) / (2 * U);
    if (npair > 0) {
      load_grp(a0, b0, c);
      for (int i = 0; i < npair - 1; ++i) {
        load_grp(a1, b1, c + U);
        mma_grp(a0, b0);
        load_grp(a0, b0, c + 2 * U);
        mma_grp(a1, b1);
        c += 2 * U;
      }
      load_grp(a1, b1, c + U);
      mma_grp(a0, b0);
      mma_grp(a1, b1);
      c += 2 * U;
    }
    for (; c < c_end; ++c) {
      const i16x8 a = __builtin_nontemporal_load(xa + c * 4);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[nt] = mfma16x16x32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, wb[(c * NT + nt) * 64]),
                               acc[nt]);
    }
  }

  if constexpr (HS > 1) {
    if (hp > 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) s_acc[(((hp - 1) * TG + tg) * NT + nt) * 64 + lane] = acc[nt];
    }
  }
  __syncthreads();  // s_cnt zeroed, partial accumulators visible
  if constexpr (HS > 1) {
    if (hp == 0) {
#pragma unroll
      for (int q = 1; q < HS; ++q)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] += s_acc[(((q - 1) * TG + tg) * NT + nt) * 64 + lane];
    }
  }

  if (hp == 0) route_group<NT>(acc, t0, lane, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt, s_p[tg],
                              &s_z[tg], &s_nf[tg]);
  __syncthreads();
  // ---- per-block partials (fixed-order sums over token groups) ----
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float p = 0.f;
#pragma unroll
    for (int q = 0; q < TG; ++q) p += s_p[q][e];
    part_cnt[(int64_t)blockIdx.x * E + e] = s_cnt[e];
    part_p[(int64_t)blockIdx.x * E + e] = p;
  }
  if (threadIdx.x == 0) {
    float z = 0.f;
    int nfs = 0;
#pragma unroll
    for (int q = 0; q < TG; ++q) {
      z += s_z[q];
      nfs += s_nf[q];
    }
    part_z[2 * blockIdx.x] = z;
    part_z[2 * blockIdx.x + 1] = (float)nfs;
  }
}


// Standalone finalize: one block; 1024 threads give each expert up to 16 loaders of its partials.
constexpr int kFinThreads = 1024;
__global__ __launch_bounds__(kFinThreads) void k_router_finalize(const int* __restrict__ part_cnt,
                                                         const float* __restrict__ part_p,
                                                         const float* __restrict__ part_z, int nblk, int N, int E,
                                                         int K, float aux_coef, float z_coef,
                                                         int64_t* __restrict__ cnt_out, float* __restrict__ stats,
                                                         float* __restrict__ aux_out, float* __restrict__ z_out) {
  __shared__ float scratch[finalize_scratch_floats<kFinThreads>()];
  router_finalize_block<kFinThreads>(part_cnt, part_p, part_z, nblk, N, E, K, aux_coef, z_coef, cnt_out, stats, aux_out, z_out,
                             scratch);
}

// ---------------------------------------------------------------------------
// Forward, streaming form (bf16 x bf16, E <= 32, H % 256 == 0).  Block = 8 waves = TG groups of 16 tokens.
// The block's 16*TG token rows are streamed through a ring of kFwdSlots LDS slots, one 256-column slice per
// slot, by LDS-DMA with whole 128-byte lines and the streaming cache policy (sc1 nt: the tokens are read
// once); the matching 256 rows of the raw gate [H, E] ride along in the same slot, so the gate needs no
// packing pass.  Wave w owns the 32-column chunk w of every slice for all TG groups: its MFMA A fragments
// are 16-byte LDS reads (x tile rows are XOR-swizzled in 16-byte units, so the 16 rows one read touches hit
// 16 different bank groups) and its B fragments are gathered from the gate rows.  The 8 partial logit tiles
// are summed in LDS in wave order, waves 0 .. TG-1 route one group each, and the block's partial statistics
// go to part_*.  The last block to finish (ticket counter: zero on entry, reset to zero by that block) folds
// all blocks' partials, so the finalize needs no launch of its own.
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void_r;
__device__ __forceinline__ uint32_t lds_addr_r(const void* p) { return (uint32_t)(uintptr_t)(lds_void_r*)p; }

// One 16-byte-per-lane LDS-DMA with the streaming cache policy.  Issued from asm so the compiler does not
// make the LDS reads of other slots wait for it; completion is ordered by explicit vmcnt waits.
__device__ __forceinline__ void lds_dma16_stream(const void* src, uint32_t lds) {
  __asm__ volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off sc1 nt" : : "v"(src), "{m0}"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void router_wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Block tail of the streaming forwards (512 threads): the block's partial statistics (fixed-order sums over
// its TG token groups) go to part_* as write-through stores, and the last block to finish (ticket counter:
// zero on entry, reset to zero by that block) folds every block's partials, so the finalize needs no launch
// of its own.  The partials are at the coherence point before the ticket increment: every thread waits for
// its own stores (s_waitcnt: a workgroup barrier alone does not wait for global stores) before the barrier
// that precedes thread 0's increment, and the last block reads them past the L2.
template <int TG, int NT>
__device__ __forceinline__ void fwd_block_tail(const int* s_cnt, const float (*s_p)[NT * 16], const float* s_z,
                                               const int* s_nf, int& s_last, float* s_fin, int N, int E, int K,
                                               int* __restrict__ part_cnt, float* __restrict__ part_p,
                                               float* __restrict__ part_z, unsigned* __restrict__ ticket,
                                               float aux_coef, float z_coef, int64_t* __restrict__ cnt_out,
                                               float* __restrict__ stats, float* __restrict__ aux_out,
                                               float* __restrict__ z_out) {
  for (int e = threadIdx.x; e < E; e += 512) {
    float p = 0.f;
#pragma unroll
    for (int q = 0; q < TG; ++q) p += s_p[q][e];
    st_part(&part_cnt[(int64_t)blockIdx.x * E + e], s_cnt[e]);
    st_part(&part_p[(int64_t)blockIdx.x * E + e], p);
  }
  if (threadIdx.x == 0) {
    float z = 0.f;
    int nfs = 0;
#pragma unroll
    for (int q = 0; q < TG; ++q) {
      z += s_z[q];
      nfs += s_nf[q];
    }
    st_part(&part_z[2 * blockIdx.x], z);
    st_part(&part_z[2 * blockIdx.x + 1], (float)nfs);
  }
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  router_finalize_block<512, true>(part_cnt, part_p, part_z, gridDim.x, N, E, K, aux_coef, z_coef, cnt_out, stats, aux_out,
                                   z_out, s_fin);
  if (threadIdx.x == 0) *ticket = 0u;
}

template <int NT, int TG>
__global__ __launch_bounds__(512) void k_router_fwd_stream(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ wg, const float* __restrict__ bias, int N, int H,
    int E, int K, int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt, float* __restrict__ logits_out,
    float* __restrict__ lse_out, int* __restrict__ part_cnt, float* __restrict__ part_p, float* __restrict__ part_z,
    unsigned* __restrict__ ticket, float aux_coef, float z_coef, int64_t* __restrict__ cnt_out,
    float* __restrict__ stats, float* __restrict__ aux_out, float* __restrict__ z_out) {
  constexpr int ROWS = 16 * TG;
  constexpr int XB = ROWS * 512;    // x tile of one slice: ROWS rows x 256 columns (bf16)
  constexpr int GI = NT;            // gate DMA instructions per wave per slice (1 KB each)
  constexpr int GB = 8 * GI * 1024; // gate tile region: 256 rows x E <= 16 * NT experts (bf16), padded
  constexpr int SLOT = XB + GB;
  constexpr int XI = ROWS / 16;     // x DMA instructions per wave per slice (2 rows x 512 B each)
  constexpr int GPS = XI + GI;      // DMA instructions per wave per slice
  // ring depth: 4 slots (3 slices in flight) fill the 160 KB LDS with NT == 1; NT == 2 fits 3
  constexpr int kFwdSlots = NT == 1 ? 4 : 3;
  static_assert(kFwdSlots <= 4, "the waits below cover at most two slices ahead");
  constexpr int RING = kFwdSlots * SLOT;
  // after the stream the ring holds the partial logit tiles and the epilogue's small arrays
  constexpr int ACC = 8 * TG * NT * 64 * 16;
  constexpr int O_CNT = ACC, O_P = O_CNT + NT * 16 * 4, O_Z = O_P + TG * NT * 16 * 4, O_NF = O_Z + TG * 4;
  constexpr int O_LAST = O_NF + TG * 4, O_FIN = O_LAST + 16;
  constexpr int O_LG = O_FIN + finalize_scratch_floats<512>() * 4;
  constexpr int O_PICK = O_LG + 16 * TG * 17 * 4;
  constexpr int EPI = O_PICK + (NT == 1 ? 64 * 4 : 0);
  static_assert(RING >= EPI, "ring too small for the epilogue arrays");
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING];
  f32x4(*s_acc)[TG][NT][64] = reinterpret_cast<f32x4(*)[TG][NT][64]>(ring);
  int* s_cnt = reinterpret_cast<int*>(ring + O_CNT);
  float(*s_p)[NT * 16] = reinterpret_cast<float(*)[NT * 16]>(ring + O_P);
  float* s_z = reinterpret_cast<float*>(ring + O_Z);
  int* s_nf = reinterpret_cast<int*>(ring + O_NF);
  int& s_last = *reinterpret_cast<int*>(ring + O_LAST);
  float* s_fin = reinterpret_cast<float*>(ring + O_FIN);

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int n = lane & 15;
  const int t0 = blockIdx.x * ROWS;

  // x DMA: instruction j (= XI*wv + q) of a slice fills rows 2j, 2j+1 (lanes 0-31 / 32-63): lane slot
  // u' = lane%32 holds the row's 16-byte unit u = u' ^ (row & 31) of the slice (rows past N re-read row N-1)
  const uint16_t* xsrc[XI];
#pragma unroll
  for (int q = 0; q < XI; ++q) {
    const int row = 2 * (XI * wv + q) + (lane >> 5);
    const int u = (lane & 31) ^ (row & 31);
    xsrc[q] = x + (int64_t)min(t0 + row, N - 1) * H + u * 8;
  }
  // gate DMA: the slice's 256 gate rows are 512*E contiguous bytes; instruction j (= GI*wv + q) copies
  // bytes [1024 j, 1024 j + 1024) of them, lanes past the end re-read the slice start (never used)
  const int gbytes = 512 * E;
  int gofs[GI];
#pragma unroll
  for (int q = 0; q < GI; ++q) {
    const int b = (GI * wv + q) * 1024 + lane * 16;
    gofs[q] = b < gbytes ? b : 0;
  }
  const int nsl = H >> 8;
  auto slot_ptr = [&](int sl) { return ring + (sl % kFwdSlots) * SLOT; };
  auto issue = [&](int sl) {
    uint8_t* const sp = slot_ptr(sl);
#pragma unroll
    for (int q = 0; q < XI; ++q) lds_dma16_stream(xsrc[q] + sl * 256, lds_addr_r(sp + (XI * wv + q) * 1024));
    const uint8_t* gsrc = reinterpret_cast<const uint8_t*>(wg) + (int64_t)sl * gbytes;
#pragma unroll
    for (int q = 0; q < GI; ++q) lds_dma16_stream(gsrc + gofs[q], lds_addr_r(sp + XB + (GI * wv + q) * 1024));
  };

  f32x4 acc[TG][NT];
#pragma unroll
  for (int q = 0; q < TG; ++q)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[q][nt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int sl = 0; sl < kFwdSlots - 1; ++sl)
    if (sl < nsl) issue(sl);
  for (int sl = 0; sl < nsl; ++sl) {
    // slice sl has landed: only the slices issued after it (min(kFwdSlots - 2, nsl - 1 - sl)) may be pending
    const int ahead = min(kFwdSlots - 2, nsl - 1 - sl);
    if (ahead >= 2) router_wait_vmcnt<2 * GPS>();
    else if (ahead == 1) router_wait_vmcnt<GPS>();
    else router_wait_vmcnt<0>();
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's part of slice sl is in LDS; every wave is done with slice sl-1
    __asm__ volatile("" ::: "memory");
    if (sl + kFwdSlots - 1 < nsl) issue(sl + kFwdSlots - 1);  // into the slot of slice sl-1
    const uint8_t* const sp = slot_ptr(sl);
    i16x8 a[TG], b[NT];
#pragma unroll
    for (int q = 0; q < TG; ++q) {
      const int row = 16 * q + n;
      const int u = 4 * wv + g;
      a[q] = *reinterpret_cast<const i16x8*>(sp + row * 512 + ((u ^ (row & 31)) << 4));
    }
    const uint16_t* gt = reinterpret_cast<const uint16_t*>(sp + XB);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int e = nt * 16 + n;
      const int ec = min(e, E - 1);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const short v = (short)gt[(32 * wv + 8 * g + j) * E + ec];
        b[nt][j] = e < E ? v : (short)0;
      }
    }
#pragma unroll
    for (int q = 0; q < TG; ++q)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[q][nt] = mfma16x16x32(__builtin_bit_cast(bf16x8, a[q]), __builtin_bit_cast(bf16x8, b[nt]), acc[q][nt]);
  }
  lds_sync();  // every wave is done with the ring: it now holds the partial logit tiles

#pragma unroll
  for (int q = 0; q < TG; ++q)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) s_acc[wv][q][nt][lane] = acc[q][nt];
  for (int i = threadIdx.x; i < NT * 16; i += 512) s_cnt[i] = 0;
  lds_sync();  // partial tiles visible, s_cnt zeroed
  if constexpr (NT == 1) {
    float* s_lg = reinterpret_cast<float*>(ring + O_LG);
    int* s_pick = reinterpret_cast<int*>(ring + O_PICK);
    const float* s_accf = reinterpret_cast<const float*>(ring);
    if (E <= 8)
      route_lanes<TG, 8>(s_accf, s_lg, s_pick, t0, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt,
                         s_p, s_z, s_nf);
    else
      route_lanes<TG, 16>(s_accf, s_lg, s_pick, t0, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt,
                          s_p, s_z, s_nf);
  } else if (wv < TG) {
    f32x4 lg[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      lg[nt] = s_acc[0][wv][nt][lane];
#pragma unroll
      for (int w = 1; w < 8; ++w) lg[nt] += s_acc[w][wv][nt][lane];
    }
    route_group<NT>(lg, t0 + 16 * wv, lane, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt, s_p[wv],
                    &s_z[wv], &s_nf[wv]);
  }
  lds_sync();  // the block's statistics are in LDS; the routing outputs' stores drain in the tail's wait
  fwd_block_tail<TG, NT>(s_cnt, s_p, s_z, s_nf, s_last, s_fin, N, E, K, part_cnt, part_p, part_z, ticket, aux_coef,
                         z_coef, cnt_out, stats, aux_out, z_out);
}

// ---------------------------------------------------------------------------
// Forward, wide streaming form (bf16 x bf16, 32 < E <= 256 as NT = 4, 8 or 16 tiles of 16 experts,
// H % 64 == 0).  With many experts the gate is as large per hidden column as a sizeable batch of token
// rows, so the block is sized to amortise it: 128 token rows per block (8 waves, one 16-token group
// each).  The block streams 64-column slices through a ring of kSlots LDS slots by LDS-DMA with the
// streaming cache policy: the x tile (128 rows x 128 bytes, 16-byte units XOR-swizzled by (row >> 1) & 7,
// so the 16 rows one fragment read touches hit distinct bank groups) and the matching two 32-row chunks
// of the gate in MFMA fragment order (k_pack_gate's layout), which ride along as one contiguous range.
// Each wave reads its A fragment and the NT B fragments as 16-byte LDS reads and accumulates its
// group's logits over the whole hidden dim in registers, so the epilogue routes straight from them.
// ---------------------------------------------------------------------------
template <int NT>
struct WideFwd {
  static constexpr int ROWS = 128;
  static constexpr int XB = ROWS * 128;  // x tile of one slice (16 KB)
  static constexpr int GB = NT * 2048;   // packed gate of one slice: 2 chunks x NT tiles x 1 KB
  static constexpr int SLOT = XB + GB;
  static constexpr int XI = XB / 8192;   // x DMA instructions per wave per slice
  static constexpr int GI = GB / 8192;   // gate DMA instructions per wave per slice
  static constexpr int GPS = XI + GI;
  // NT == 4: 3 slots (72 KB) let two blocks share a CU, so one block's routing overlaps the other's stream
  static constexpr int kSlots = NT == 4 ? 3 : (NT == 8 ? 4 : 3);
};

template <int GPS>
__device__ __forceinline__ void wide_wait(int ahead) {
  // at most `ahead` later slices (GPS DMA instructions each) may still be in flight
  switch (ahead) {
    case 0: router_wait_vmcnt<0>(); break;
    case 1: router_wait_vmcnt<GPS>(); break;
    case 2: router_wait_vmcnt<2 * GPS>(); break;
    case 3: router_wait_vmcnt<3 * GPS>(); break;
    default: router_wait_vmcnt<4 * GPS>(); break;
  }
}

template <int NT>
__global__ __launch_bounds__(512) void k_router_fwd_wide(
    const uint16_t* __restrict__ x, const i16x8* __restrict__ wp, const float* __restrict__ bias, int N, int H,
    int E, int K, int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt, float* __restrict__ logits_out,
    float* __restrict__ lse_out, int* __restrict__ part_cnt, float* __restrict__ part_p, float* __restrict__ part_z,
    unsigned* __restrict__ ticket, float aux_coef, float z_coef, int64_t* __restrict__ cnt_out,
    float* __restrict__ stats, float* __restrict__ aux_out, float* __restrict__ z_out) {
  using P = WideFwd<NT>;
  constexpr int TG = 8;
  static_assert(P::kSlots - 2 <= 4, "wide_wait covers at most four slices ahead");
  constexpr int RING = P::kSlots * P::SLOT;
  // after the stream the ring holds the epilogue's small arrays
  constexpr int O_CNT = 0, O_P = O_CNT + NT * 16 * 4, O_Z = O_P + TG * NT * 16 * 4, O_NF = O_Z + TG * 4;
  constexpr int O_LAST = O_NF + TG * 4, O_FIN = O_LAST + 16;
  constexpr int EPI = O_FIN + finalize_scratch_floats<512>() * 4;
  // NT <= 8: each wave's routing tile (16 rows of NT*16 + 4 floats) after the epilogue arrays
  constexpr int O_TR = (EPI + 15) & ~15, TRB = 16 * (NT * 16 + 4) * 4;
  static_assert(RING >= (NT <= 8 ? O_TR + TG * TRB : EPI), "ring too small for the epilogue arrays");
  __shared__ __attribute__((aligned(16))) uint8_t ring[RING];
  int* s_cnt = reinterpret_cast<int*>(ring + O_CNT);
  float(*s_p)[NT * 16] = reinterpret_cast<float(*)[NT * 16]>(ring + O_P);
  float* s_z = reinterpret_cast<float*>(ring + O_Z);
  int* s_nf = reinterpret_cast<int*>(ring + O_NF);
  int& s_last = *reinterpret_cast<int*>(ring + O_LAST);
  float* s_fin = reinterpret_cast<float*>(ring + O_FIN);

  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4;
  const int n = lane & 15;
  const int t0 = blockIdx.x * P::ROWS;

  // x DMA: instruction j (= XI*wv + q) of a slice fills rows 8j .. 8j+7; lane l writes row 8j + l/8, LDS
  // unit l%8, which holds the row's 16-byte unit (l%8) ^ ((row >> 1) & 7) (rows past N re-read row N-1)
  const uint16_t* xsrc[P::XI];
#pragma unroll
  for (int q = 0; q < P::XI; ++q) {
    const int row = 8 * (P::XI * wv + q) + (lane >> 3);
    const int u = (lane & 7) ^ ((row >> 1) & 7);
    xsrc[q] = x + (int64_t)min(t0 + row, N - 1) * H + u * 8;
  }
  const uint8_t* gsrc = reinterpret_cast<const uint8_t*>(wp) + (P::GI * wv) * 1024 + lane * 16;
  const int nsl = H >> 6;
  auto slot_ptr = [&](int sl) { return ring + (sl % P::kSlots) * P::SLOT; };
  auto issue = [&](int sl) {
    uint8_t* const sp = slot_ptr(sl);
#pragma unroll
    for (int q = 0; q < P::XI; ++q) lds_dma16_stream(xsrc[q] + sl * 64, lds_addr_r(sp + (P::XI * wv + q) * 1024));
#pragma unroll
    for (int q = 0; q < P::GI; ++q)
      lds_dma16_stream(gsrc + (int64_t)sl * P::GB + q * 1024, lds_addr_r(sp + P::XB + (P::GI * wv + q) * 1024));
  };

  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int sl = 0; sl < P::kSlots - 1; ++sl)
    if (sl < nsl) issue(sl);
  const int arow = 16 * wv + n;  // this lane's A row in the x tile
  for (int sl = 0; sl < nsl; ++sl) {
    wide_wait<P::GPS>(min(P::kSlots - 2, nsl - 1 - sl));
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave's part of slice sl is in LDS; every wave is done with slice sl-1
    __asm__ volatile("" ::: "memory");
    if (sl + P::kSlots - 1 < nsl) issue(sl + P::kSlots - 1);  // into the slot of slice sl-1
    const uint8_t* const sp = slot_ptr(sl);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const i16x8 a = *reinterpret_cast<const i16x8*>(sp + arow * 128 + (((4 * h + g) ^ ((arow >> 1) & 7)) << 4));
      const i16x8* gt = reinterpret_cast<const i16x8*>(sp + P::XB) + h * NT * 64 + lane;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[nt] = mfma16x16x32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, gt[nt * 64]), acc[nt]);
    }
  }
  __syncthreads();  // every wave is done with the ring

  for (int i = threadIdx.x; i < NT * 16; i += 512) s_cnt[i] = 0;
  __syncthreads();
  if constexpr (NT <= 8) {
    float* tile = reinterpret_cast<float*>(ring + O_TR + wv * TRB);
    route_quad<NT>(acc, tile, t0 + 16 * wv, lane, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt,
                   s_p[wv], &s_z[wv], &s_nf[wv]);
  } else {
    route_group<NT>(acc, t0 + 16 * wv, lane, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt,
                    s_p[wv], &s_z[wv], &s_nf[wv]);
  }
  __syncthreads();
  fwd_block_tail<TG, NT>(s_cnt, s_p, s_z, s_nf, s_last, s_fin, N, E, K, part_cnt, part_p, part_z, ticket, aux_coef,
                         z_coef, cnt_out, stats, aux_out, z_out);
}

// ---------------------------------------------------------------------------
// Forward, fp32 x and fp32 gate (E <= 64, H % 4 == 0, x 16-byte aligned).  The gate GEMM runs on
// v_mfma_f32_16x16x4_f32 (fp32 products, fp32 sums), whose 16x16 accumulator layout is the one the bf16
// kernels route from.  Block = 8 waves = TG groups of 16 tokens x HS = 8 / TG waves per group; wave hp of a
// group sums its logits over the hp-th contiguous 1/HS of the 16-column chunks of the hidden dim.  Per chunk
// c, lane l reads x[t0 + l % 16][k .. k + 3] with one 16-byte load (k = 16 c + 4 (l / 16)) and feeds the four
// values to four MFMAs together with the gate rows k .. k + 3 of its expert column l % 16: in MFMA s, the
// k slot l / 16 holds k + s for A and for B alike, which is all the product needs.  The HS partial tiles are
// summed in LDS in wave order, wave hp = 0 of each group routes it (route_group), and the block tail
// publishes the block's statistics and folds every block's in the last block to finish.
// ---------------------------------------------------------------------------
template <int NT, int TG>
__global__ __launch_bounds__(512) void k_router_fwd_f32(
    const float* __restrict__ x, const float* __restrict__ wg, const float* __restrict__ bias, int N, int H, int E,
    int K, int64_t* __restrict__ idx_out, void* __restrict__ w_out, int w_dt, float* __restrict__ logits_out,
    float* __restrict__ lse_out, int* __restrict__ part_cnt, float* __restrict__ part_p, float* __restrict__ part_z,
    unsigned* __restrict__ ticket, float aux_coef, float z_coef, int64_t* __restrict__ cnt_out,
    float* __restrict__ stats, float* __restrict__ aux_out, float* __restrict__ z_out) {
  constexpr int HS = 8 / TG;
  constexpr int U = 4;  // chunks per load group
  __shared__ f32x4 s_acc[(HS > 1 ? HS - 1 : 1) * TG * NT * 64];
  __shared__ int s_cnt[NT * 16];
  __shared__ float s_p[TG][NT * 16];
  __shared__ float s_z[TG];
  __shared__ int s_nf[TG];
  __shared__ int s_last;
  __shared__ float s_fin[finalize_scratch_floats<512>()];

  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int tg = wv / HS;
  const int hp = wv % HS;
  const int n = lane & 15;
  const int q = lane >> 4;
  const int t0 = blockIdx.x * (16 * TG) + tg * 16;
  for (int i = threadIdx.x; i < NT * 16; i += 512) s_cnt[i] = 0;

  const int row = min(t0 + n, N - 1);
  const float* xr = x + (int64_t)row * H + 4 * q;
  const int nc = (H + 15) / 16;   // chunks; all but a last partial one (H % 16 != 0) lie inside the row
  const int nfull = H / 16;
  const int per = (nc + HS - 1) / HS;
  const int c_beg = min(nc, hp * per);
  const int c_end = min(nc, c_beg + per);

  f32x4 acc[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  // gate row k + s of expert column nt * 16 + n (zero past E or past H)
  auto gate = [&](int k, int s, int nt) -> float {
    const int e = nt * 16 + n;
    return (e < E && k + s < H) ? wg[(int64_t)(k + s) * E + e] : 0.f;
  };
  auto chunk_mma = [&](const f32x4& a, const float (&b)[NT][4]) {
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s2], b[nt][s2], acc[nt], 0, 0, 0);
  };
  if (t0 < N) {
    const int c_mid = min(c_end, nfull);
    int c = c_beg;
    for (; c + U <= c_mid; c += U) {
      f32x4 a[U];
      float b[U][NT][4];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        a[u] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(xr + (c + u) * 16));
        const int k = (c + u) * 16 + 4 * q;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int s2 = 0; s2 < 4; ++s2) b[u][nt][s2] = gate(k, s2, nt);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) chunk_mma(a[u], b[u]);
    }
    for (; c < c_end; ++c) {  // the rest, and the last partial chunk (lanes past H read zeros)
      const int k = c * 16 + 4 * q;
      const f32x4 a = k < H ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(xr + c * 16))
                            : f32x4{0.f, 0.f, 0.f, 0.f};
      float b[NT][4];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2) b[nt][s2] = gate(k, s2, nt);
      chunk_mma(a, b);
    }
  }

  if constexpr (HS > 1) {
    if (hp > 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) s_acc[(((hp - 1) * TG + tg) * NT + nt) * 64 + lane] = acc[nt];
    }
  }
  __syncthreads();  // s_cnt zeroed, partial tiles visible
  if constexpr (HS > 1) {
    if (hp == 0) {
#pragma unroll
      for (int q2 = 1; q2 < HS; ++q2)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt] += s_acc[(((q2 - 1) * TG + tg) * NT + nt) * 64 + lane];
    }
  }
  if (hp == 0) route_group<NT>(acc, t0, lane, bias, N, E, K, idx_out, w_out, w_dt, logits_out, lse_out, s_cnt, s_p[tg],
                              &s_z[tg], &s_nf[tg]);
  __syncthreads();
  fwd_block_tail<TG, NT>(s_cnt, s_p, s_z, s_nf, s_last, s_fin, N, E, K, part_cnt, part_p, part_z, ticket, aux_coef,
                         z_coef, cnt_out, stats, aux_out, z_out);
}

// ---------------------------------------------------------------------------
// Generic forward: logits by VALU (one wave per token), then route_from_logits.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_logits_generic(const void* __restrict__ x, int x_dt,
                                                        const void* __restrict__ wg, int w_dt,
                                                        const float* __restrict__ bias, int N, int H, int E,
                                                        float* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int wpb = blockDim.x >> 6;
  for (int t = blockIdx.x * wpb + (threadIdx.x >> 6); t < N; t += gridDim.x * wpb) {
    for (int e0 = 0; e0 < E; e0 += 16) {
      float acc[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[j] = 0.f;
      for (int h = lane; h < H; h += 64) {
        const float xv = load_f(x, x_dt, (int64_t)t * H + h);
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (e0 + j < E) acc[j] = fmaf(xv, load_f(wg, w_dt, (int64_t)h * E + e0 + j), acc[j]);
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float v = wave_sum(acc[j]);
        if (lane == 0 && e0 + j < E) logits[(int64_t)t * E + e0 + j] = v + (bias ? bias[e0 + j] : 0.f);
      }
    }
  }
}

// One wave per token; lane holds experts lane, lane+64, lane+128, lane+192.
__global__ __launch_bounds__(256) void k_route_from_logits(const float* __restrict__ logits, int N, int E, int K,
                                                           int tok_per_blk, int64_t* __restrict__ idx_out,
                                                           void* __restrict__ w_out, int w_dt,
                                                           float* __restrict__ lse_out, int* __restrict__ part_cnt,
                                                           float* __restrict__ part_p, float* __restrict__ part_z) {
  __shared__ int s_cnt[kMaxE];
  __shared__ float s_p[4][kMaxE];
  __shared__ float s_z[4];
  __shared__ int s_nf[4];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  int nf = 0;
  for (int i = threadIdx.x; i < kMaxE; i += blockDim.x) s_cnt[i] = 0;
  __syncthreads();
  float pacc[4] = {0.f, 0.f, 0.f, 0.f};
  float zacc = 0.f;
  const int tbeg = blockIdx.x * tok_per_blk;
  const int tend = min(N, tbeg + tok_per_blk);
  for (int t = tbeg + wv; t < tend; t += 4) {
    float lg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = lane + 64 * j;
      float v = (e < E) ? logits[(int64_t)t * E + e] : -INFINITY;
      if (e < E && !isfinite(v)) ++nf;
      if (v != v) v = -INFINITY;
      lg[j] = v;
    }
    const float m = wave_max(fmaxf(fmaxf(lg[0], lg[1]), fmaxf(lg[2], lg[3])));
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) s += expf(lg[j] - m);
    s = wave_sum(s);
    const float inv = 1.f / s;
    const float lse = m + logf(s);
    if (lane == 0) lse_out[t] = lse;
    zacc += lse * lse;
#pragma unroll
    for (int j = 0; j < 4; ++j) pacc[j] += expf(lg[j] - m) * inv;
    uint32_t sel = 0;
    int my_e = 0;
    float my_p = 0.f;
    float psum = 0.f;
    for (int r = 0; r < K; ++r) {
      float bv = -INFINITY;
      int be = 0x7fffffff;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        if (e < E && !((sel >> j) & 1u) && better(lg[j], e, bv, be)) {
          bv = lg[j];
          be = e;
        }
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oe = __shfl_xor(be, o);
        if (better(ov, oe, bv, be)) {
          bv = ov;
          be = oe;
        }
      }
      if ((be & 63) == lane) sel |= 1u << (be >> 6);
      const float pv = expf(bv - m) * inv;
      psum += pv;
      if (r == lane) {
        my_e = be;
        my_p = pv;
      }
    }
    const float rden = 1.f / fmaxf(psum, 1e-30f);
    if (lane < K) {
      idx_out[(int64_t)t * K + lane] = my_e;
      store_f(w_out, w_dt, (int64_t)t * K + lane, my_p * rden);
      atomicAdd(&s_cnt[my_e], 1);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int e = lane + 64 * j;
    if (e < E) s_p[wv][e] = pacc[j];
  }
  nf = wave_sum(nf);
  if (lane == 0) {
    s_z[wv] = zacc;
    s_nf[wv] = nf;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    part_cnt[(int64_t)blockIdx.x * E + e] = s_cnt[e];
    part_p[(int64_t)blockIdx.x * E + e] = ((s_p[0][e] + s_p[1][e]) + s_p[2][e]) + s_p[3][e];
  }
  if (threadIdx.x == 0) {
    part_z[2 * blockIdx.x] = ((s_z[0] + s_z[1]) + s_z[2]) + s_z[3];
    part_z[2 * blockIdx.x + 1] = (float)(s_nf[0] + s_nf[1] + s_nf[2] + s_nf[3]);
  }
}

// ---------------------------------------------------------------------------
// Backward 1: G = dL/dlogits.  LPT lanes per token (EPL experts per lane).
// Writes G (f32) and, when gb != nullptr, G rounded to bf16 in a zero-padded
// [N, ekp] layout.
// ---------------------------------------------------------------------------
// dL/dlogits of one token, LPT lanes per token, lane `sub` owning experts sub + LPT*j (j < EPL):
//   softmax p, renormalised top-k weights v_k = p_{e_k} / max(sum_k p_{e_k}, 1e-30) with upstream gw,
//   aux term ca * p (f - sum p f) with f_e = cnt_e / (N K), z term cz * lse * p.
// The exponentials, the logarithm and the reciprocals take the hardware forms (v_exp_f32, v_log_f32,
// v_rcp_f32: relative error ~1e-6 at these magnitudes, far below the bf16 rounding G gets before its
// products): the full-precision library forms expand to ~15 instructions each, and in the backward's
// prologue, run once per block on a cold instruction cache, code length is time.
struct GCoef {
  float ca, cz, inv_nk;
};

__device__ __forceinline__ GCoef glogit_coef(const float* __restrict__ grad_aux, const float* __restrict__ grad_z,
                                             float aux_coef, float z_coef, int N, int E, int K) {
  const float ga = grad_aux ? grad_aux[0] : 1.f;
  const float gz = grad_z ? grad_z[0] : 1.f;
  return GCoef{aux_coef * ga * (float)E / (float)N, z_coef * gz * 2.f / (float)N, 1.f / ((float)N * (float)K)};
}

// Sum / max over the LPT lanes that share a token (DPP within a row of 16 lanes).
template <int LPT>
__device__ __forceinline__ float grp_sum(float v) {
  if constexpr (LPT == 16) {
    return row16_sum(v);
  } else {
#pragma unroll
    for (int o = LPT / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
  }
}
template <int LPT>
__device__ __forceinline__ float grp_max(float v) {
  if constexpr (LPT == 16) {
    return row16_max(v);
  } else {
#pragma unroll
    for (int o = LPT / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
  }
}

template <int LPT, int EPL>
__device__ __forceinline__ void glogit_token(const float* __restrict__ logits, const int64_t* __restrict__ idx,
                                             const void* __restrict__ gw, int gw_dt,
                                             const int64_t* __restrict__ cnt, const GCoef& c, int t, int E, int K,
                                             int sub, float (&gl)[EPL]) {
  float lg[EPL], p[EPL], f[EPL], gp[EPL];
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    const int e = sub + LPT * j;
    lg[j] = (e < E) ? logits[(int64_t)t * E + e] : -INFINITY;
    f[j] = (e < E && c.ca != 0.f) ? (float)cnt[e] * c.inv_nk : 0.f;
    gp[j] = 0.f;
  }
  float m = lg[0];
#pragma unroll
  for (int j = 1; j < EPL; ++j) m = fmaxf(m, lg[j]);
  m = grp_max<LPT>(m);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    p[j] = __expf(lg[j] - m);
    s += p[j];
  }
  s = grp_sum<LPT>(s);
  const float inv = __builtin_amdgcn_rcpf(s);
  const float lse = m + __logf(s);
#pragma unroll
  for (int j = 0; j < EPL; ++j) p[j] *= inv;
  // With K == 1 the renormalised weight is v / v = 1 (the top-1 probability is at least 1/E), so no gradient
  // reaches the logits through it: the term is skipped rather than formed as a difference of rounded equals.
  if (gw != nullptr && K > 1) {
    // S = max(sum v, 1e-30); gwv = sum gw*v; grad_v = gw/S - gwv/S^2
    // v_k = p[e_k], picked from this lane's registers (the lane holding e_k contributes, the row sums)
    float S = 0.f, gwv = 0.f;
    for (int k = 0; k < K; ++k) {
      const int e = (int)idx[(int64_t)t * K + k];
      float v = 0.f;
#pragma unroll
      for (int j = 0; j < EPL; ++j) v = (e == sub + LPT * j) ? p[j] : v;
      v = grp_sum<LPT>(v);
      const float gk = load_f(gw, gw_dt, (int64_t)t * K + k);
      S += v;
      gwv += gk * v;
    }
    S = fmaxf(S, 1e-30f);
    const float iS = __builtin_amdgcn_rcpf(S);
    for (int k = 0; k < K; ++k) {
      const int e = (int)idx[(int64_t)t * K + k];
      const float gk = load_f(gw, gw_dt, (int64_t)t * K + k);
      const float gv = gk * iS - gwv * iS * iS;
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (e == sub + LPT * j) gp[j] += gv;
    }
  }
  float inner = 0.f, pf = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    inner += gp[j] * p[j];
    pf += p[j] * f[j];
  }
  inner = grp_sum<LPT>(inner);
  pf = grp_sum<LPT>(pf);
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    float v = p[j] * (gp[j] - inner);
    if (c.ca != 0.f) v += c.ca * p[j] * (f[j] - pf);
    if (c.cz != 0.f) v += c.cz * lse * p[j];
    gl[j] = v;
  }
}

// G of one token from values already in registers (one lane per token): lg[e] = the token's logits (-inf past
// E), f[e] = its expert's dispatch fraction (cnt * inv_nk; 0 without the aux term), and the token's top-k ids and
// upstream weight gradients (K <= KR).  The same arithmetic as glogit_token<1, EPL>.
template <int EPL, int KR>
__device__ __forceinline__ void glogit_token_regs(const float (&lg)[EPL], const float (&f)[EPL], const int (&ik)[KR],
                                                  const float (&gk)[KR], bool has_gw, const GCoef& c, int K,
                                                  float (&gl)[EPL]) {
  float p[EPL], gp[EPL];
  float m = lg[0];
#pragma unroll
  for (int j = 1; j < EPL; ++j) m = fmaxf(m, lg[j]);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    p[j] = __expf(lg[j] - m);
    s += p[j];
    gp[j] = 0.f;
  }
  const float inv = __builtin_amdgcn_rcpf(s);
  const float lse = m + __logf(s);
#pragma unroll
  for (int j = 0; j < EPL; ++j) p[j] *= inv;
  if (has_gw && K > 1) {  // K == 1: the renormalised weight is identically 1 (see glogit_token)
    float v[KR], S = 0.f, gwv = 0.f;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
      float vk = 0.f;
#pragma unroll
      for (int j = 0; j < EPL; ++j) vk = (ik[k] == j) ? p[j] : vk;
      v[k] = k < K ? vk : 0.f;
      S += v[k];
      gwv += (k < K ? gk[k] : 0.f) * v[k];
    }
    S = fmaxf(S, 1e-30f);
    const float iS = __builtin_amdgcn_rcpf(S);
#pragma unroll
    for (int k = 0; k < KR; ++k) {
      const float gv = gk[k] * iS - gwv * iS * iS;
#pragma unroll
      for (int j = 0; j < EPL; ++j)
        if (k < K && ik[k] == j) gp[j] += gv;
    }
  }
  float inner = 0.f, pf = 0.f;
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    inner += gp[j] * p[j];
    pf += p[j] * f[j];
  }
#pragma unroll
  for (int j = 0; j < EPL; ++j) {
    float v = p[j] * (gp[j] - inner);
    if (c.ca != 0.f) v += c.ca * p[j] * (f[j] - pf);
    if (c.cz != 0.f) v += c.cz * lse * p[j];
    gl[j] = v;
  }
}


// ---------------------------------------------------------------------------
// Backward 1: G = dL/dlogits.  LPT lanes per token (EPL experts per lane).
// Writes G (f32) and, when gb != nullptr, G rounded to bf16 in a zero-padded
// [N, ekp] layout.
// ---------------------------------------------------------------------------
template <int LPT, int EPL>
__global__ __launch_bounds__(256) void k_router_glogits(const float* __restrict__ logits,
                                                        const int64_t* __restrict__ idx, const void* __restrict__ gw,
                                                        int gw_dt, const int64_t* __restrict__ cnt,
                                                        const float* __restrict__ grad_aux,
                                                        const float* __restrict__ grad_z, float aux_coef,
                                                        float z_coef, int N, int E, int K, int round_bf16,
                                                        float* __restrict__ G, uint16_t* __restrict__ gb, int ekp) {
  constexpr int TPW = 64 / LPT;  // tokens per wave
  const int lane = threadIdx.x & 63;
  const int sub = lane % LPT;
  const int slot = lane / LPT;
  const int wpb = blockDim.x >> 6;
  const GCoef c = glogit_coef(grad_aux, grad_z, aux_coef, z_coef, N, E, K);
  const int stride = gridDim.x * wpb * TPW;
  for (int tb = (blockIdx.x * wpb + (threadIdx.x >> 6)) * TPW; tb < N; tb += stride) {
    const int t_raw = tb + slot;
    const bool valid = t_raw < N;
    const int t = valid ? t_raw : N - 1;
    float gl[EPL];
    glogit_token<LPT, EPL>(logits, idx, gw, gw_dt, cnt, c, t, E, K, sub, gl);
    if (valid) {
#pragma unroll
      for (int j = 0; j < EPL; ++j) {
        const int e = sub + LPT * j;
        if (e < E) {
          float v = gl[j];
          if (round_bf16) v = bf2f(f2bf(v));
          if (G) G[(int64_t)t * E + e] = v;
          if (gb) gb[(int64_t)t * ekp + e] = f2bf(v);
        }
      }
      if (gb) {
        for (int e = E + sub; e < ekp; e += LPT) gb[(int64_t)t * ekp + e] = 0;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward 2 (bf16 x bf16): dx = G wg^T, dwg partial = x^T G, MFMA.
// Block = 4 waves = 256 hidden columns; grid = (token chunks, H / 256).
// EK = ekp / 32 (expert k-chunks for dx), NTE = ceil(E / 16) (expert tiles
// for dwg).
// ---------------------------------------------------------------------------
constexpr int kBwdTS = 32;      // tokens per step
constexpr int kXPitch = 264;    // bf16 elements per LDS row of the x / dx tiles
template <int EK, int NTE>
__global__ __launch_bounds__(256) void k_router_dxdw_bf16(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wg,
                                                          const uint16_t* __restrict__ gb, int N, int H, int E,
                                                          int tc_len, uint16_t* __restrict__ dx,
                                                          float* __restrict__ ws_dw) {
  constexpr int EKP = EK * 32;
  constexpr int GP = EKP + 8;          // row pitch of the token-major G tile
  constexpr int GTP = kBwdTS + 8;      // row pitch of the expert-major G tile
  __shared__ __attribute__((aligned(16))) uint16_t xs[kBwdTS * kXPitch];
  __shared__ __attribute__((aligned(16))) uint16_t dxs[kBwdTS * kXPitch];
  __shared__ __attribute__((aligned(16))) uint16_t gs[kBwdTS * GP];
  __shared__ __attribute__((aligned(16))) uint16_t gts[NTE * 16 * GTP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int hb0 = blockIdx.y * 256;
  const int wcol0 = hb0 + wv * 64;  // this wave's first hidden column
  const bool wave_active = wcol0 < H;
  const int tbeg = blockIdx.x * tc_len;
  const int tend = min(N, tbeg + tc_len);

  for (int i = tid; i < NTE * 16 * GTP; i += 256) gts[i] = 0;

  // gate fragments for dx (B operand: B[k=e][n=h] = wg[h][e]), loaded once.
  i16x8 wB[4][EK];
#pragma unroll
  for (int nc = 0; nc < 4; ++nc) {
    const int h = wcol0 + nc * 16 + n;
#pragma unroll
    for (int ek = 0; ek < EK; ++ek) {
      i16x8 v;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = ek * 32 + g * 8 + j;
        v[j] = (wave_active && h < H && e < E) ? (short)wg[(int64_t)h * E + e] : (short)0;
      }
      wB[nc][ek] = v;
    }
  }

  f32x4 accw[4][NTE];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ne = 0; ne < NTE; ++ne) accw[mt][ne] = f32x4{0.f, 0.f, 0.f, 0.f};

  // x tile load mapping: 32 rows x 256 cols = 1024 chunks of 8 bf16; 4 per thread.
  u32x4 xr[4];
  auto load_x = [&](int ts0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = tid + 256 * j;
      const int r = q >> 5;
      const int col = hb0 + (q & 31) * 8;
      const int t = ts0 + r;
      if (t < tend && col < H)
        xr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + (int64_t)t * H + col));
      else
        xr[j] = u32x4{0u, 0u, 0u, 0u};
    }
  };
  if (tbeg < tend) load_x(tbeg);

  for (int ts0 = tbeg; ts0 < tend; ts0 += kBwdTS) {
    lds_sync();  // previous step done with xs / dxs / gs / gts (global prefetch and dx stores stay in flight)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = tid + 256 * j;
      const int r = q >> 5;
      *reinterpret_cast<u32x4*>(&xs[r * kXPitch + (q & 31) * 8]) = xr[j];
    }
    // G tile (bf16): token-major gs[t][e] and expert-major gts[e][t]
    for (int q = tid; q < kBwdTS * EKP; q += 256) {
      const int r = q / EKP;
      const int e = q % EKP;
      const int t = ts0 + r;
      const uint16_t v = (t < tend) ? gb[(int64_t)t * EKP + e] : (uint16_t)0;
      gs[r * GP + e] = v;
      if (e < NTE * 16) gts[e * GTP + r] = v;
    }
    if (ts0 + kBwdTS < tend) load_x(ts0 + kBwdTS);
    lds_sync();

    if (wave_active) {
      // ---- dwg partial: D[m=h][n=e] += sum_t x[t][h] G[t][e] ----
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int col = wv * 64 + mt * 16 + n;
        i16x8 a;
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = (short)xs[(g * 8 + j) * kXPitch + col];
#pragma unroll
        for (int ne = 0; ne < NTE; ++ne) {
          const i16x8 b = *reinterpret_cast<const i16x8*>(&gts[(ne * 16 + n) * GTP + g * 8]);
          accw[mt][ne] =
              mfma16x16x32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), accw[mt][ne]);
        }
      }
      // ---- dx: D[m=t][n=h] = sum_e G[t][e] wg[h][e] ----
#pragma unroll
      for (int mk = 0; mk < 2; ++mk) {
        i16x8 a[EK];
#pragma unroll
        for (int ek = 0; ek < EK; ++ek)
          a[ek] = *reinterpret_cast<const i16x8*>(&gs[(mk * 16 + n) * GP + ek * 32 + g * 8]);
#pragma unroll
        for (int nc = 0; nc < 4; ++nc) {
          f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ek = 0; ek < EK; ++ek)
            d = mfma16x16x32(__builtin_bit_cast(bf16x8, a[ek]), __builtin_bit_cast(bf16x8, wB[nc][ek]), d);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            dxs[(mk * 16 + g * 4 + i) * kXPitch + wv * 64 + nc * 16 + n] = f2bf(d[i]);
        }
      }
    }
    lds_sync();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = tid + 256 * j;
      const int r = q >> 5;
      const int col = hb0 + (q & 31) * 8;
      const int t = ts0 + r;
      if (t < tend && col < H)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(&dxs[r * kXPitch + (q & 31) * 8]),
                                    reinterpret_cast<u32x4*>(dx + (int64_t)t * H + col));
    }
  }

  if (wave_active) {
    float* out = ws_dw + (int64_t)blockIdx.x * H * E;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int ne = 0; ne < NTE; ++ne)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int h = wcol0 + mt * 16 + g * 4 + i;
          const int e = ne * 16 + n;
          if (h < H && e < E) out[(int64_t)h * E + e] = accw[mt][ne][i];
        }
  }
}

// ---------------------------------------------------------------------------
// Backward 2, streaming form (bf16 x bf16, E <= 32, H % 256 == 0): dx = G wg^T and the dwg partial
// x^T G of one (token chunk, 256 hidden columns) block.  Each wave owns 64 hidden columns and a private
// LDS tile, so after the chunk's G has been staged (token-major and expert-major) the token loop has no
// workgroup barrier: per 32-token step the wave writes its x tile to LDS, reads the dwg A operand with
// transposing reads, forms dx with MFMA into the same tile and stores it as 128-byte row segments.  x is
// prefetched two steps ahead with clamped (branch-free) loads; rows past the chunk read as zero.
// ---------------------------------------------------------------------------
constexpr int kSTC = 256;   // max tokens per chunk (a multiple of 64)
constexpr int kGRegK = 4;   // top-k widths whose ids and upstream gradients the streaming backward preloads
constexpr int kSXP = 72;    // pitch (bf16) of a wave's 32 x 64 tile: 144 bytes, conflict-free for the reads below
typedef short sh4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) sh4 lds_sh4;

// KR: top-k slots whose ids and upstream gradients are preloaded (K <= KR <= kGRegK; K > kGRegK reads them
// where G is formed).  WPB: waves per block (64 hidden columns each), 4 or 16; with 16 one block fills a CU's
// 16 wave slots, so the CU's memory requests come from one block whose waves start together (with four
// 4-wave blocks per CU the first-dispatched block's requests are served first and the others start late).
template <int NTE, int EL, int KR, int WPB>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(NTE == 1 ? 4 : 1))) void k_router_dxdw_stream(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ wg,
                                                            const float* __restrict__ logits,
                                                            const int64_t* __restrict__ idx,
                                                            const void* __restrict__ gw, int gw_dt,
                                                            const int64_t* __restrict__ cnt,
                                                            const float* __restrict__ grad_aux,
                                                            const float* __restrict__ grad_z, float aux_coef,
                                                            float z_coef, int N, int H, int E, int K, int tc_len,
                                                            int nht, uint16_t* __restrict__ dx,
                                                            const uint16_t* __restrict__ dx_add,
                                                            float* __restrict__ ws_dw, uint16_t* __restrict__ g_out,
                                                            int g_pitch) {
  constexpr int GS = NTE * 16;       // expert slots of a token-major G row
  constexpr int GP = GS + 8;         // its pitch: 16 rows of one 16-byte read hit distinct bank groups
  constexpr int GTP = kSTC + 8;      // expert-major G row pitch
  __shared__ __attribute__((aligned(16))) uint16_t gs[kSTC * GP];
  __shared__ __attribute__((aligned(16))) uint16_t gts[NTE * 16 * GTP];
  __shared__ __attribute__((aligned(16))) uint16_t xs[WPB][32 * kSXP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int chunk = blockIdx.x / nht;
  const int ht = blockIdx.x - chunk * nht;
  const int tbeg = chunk * tc_len;
  const int tend = min(N, tbeg + tc_len);
  const int nst = ((tend - tbeg + 63) / 64) * 2;  // 32-token steps, rounded up to even
  const int col0 = ht * (64 * WPB) + wv * 64;     // this wave's first hidden column
  uint16_t* xsw = xs[wv];

  // x stream: lane loads rows (lane/8) + 8j of the step, 16-byte chunk lane%8 of the wave's 64 columns
  // (rows past the chunk re-read its last row and are zeroed when written to LDS)
  const uint16_t* xw = x + col0 + (lane & 7) * 8;
  auto load_x = [&](u32x4(&r)[4], int ts0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = ts0 + (lane >> 3) + 8 * j;
      r[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xw + (int64_t)min(t, tend - 1) * H));
    }
  };
  // the same rows of an [N, H] bf16 tensor (the dx addend), same clamping
  auto load_rows = [&](const uint16_t* src, u32x4(&r)[4], int ts0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = ts0 + (lane >> 3) + 8 * j;
      r[j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(src + col0 + (lane & 7) * 8 + (int64_t)min(t, tend - 1) * H));
    }
  };
  // ---- G = dL/dlogits of the chunk, one token per thread, rounded to bf16 as the reference does
  // (grad_logits.to(tokens.dtype)) and staged in both layouts; rows past the chunk are 0.  The token's
  // logits, top-k ids and upstream gradients are requested first (clamped, branch-free loads), then the x
  // prefetch, so the small loads are not queued behind the stream; with K > kGRegK the loads happen
  // inside glogit_token instead. ----
  // EL (<= NTE * 16): experts a token's G is computed over (8 when E <= 8)
  const GCoef cf = glogit_coef(grad_aux, grad_z, aux_coef, z_coef, N, E, K);
  const int r = tid;  // blockDim == kSTC >= the chunk's rounded-up row count
  const int t = tbeg + r;
  const int tc = min(t, tend - 1);
  const bool regs = KR == 2 || K <= KR;  // the KR == 2 form is only launched with K <= 2
  // raw loads only (no conversion of a loaded value before the x prefetch is issued: using one would wait
  // for it here); the branches are wave-uniform
  float lgv[EL];
  int ikv[KR];
  uint32_t gkraw[KR];
  const bool gw16 = gw_dt == MOE_BF16;
  if (regs && wv < kSTC / 64) {  // the G waves (one token per thread)
#pragma unroll
    for (int e = 0; e < EL; ++e) lgv[e] = logits[(int64_t)tc * E + min(e, E - 1)];
#pragma unroll
    for (int k = 0; k < KR; ++k) ikv[k] = (int)idx[(int64_t)tc * K + min(k, K - 1)];
    if (gw != nullptr && gw16) {
#pragma unroll
      for (int k = 0; k < KR; ++k) gkraw[k] = static_cast<const uint16_t*>(gw)[(int64_t)tc * K + min(k, K - 1)];
    } else if (gw != nullptr) {
#pragma unroll
      for (int k = 0; k < KR; ++k) gkraw[k] = static_cast<const uint32_t*>(gw)[(int64_t)tc * K + min(k, K - 1)];
    } else {
#pragma unroll
      for (int k = 0; k < KR; ++k) gkraw[k] = 0u;
    }
  }
  u32x4 xa[4], xb[4];
  load_x(xa, tbeg);
  load_x(xb, tbeg + 32);
  {
    float gl[EL];
    if (t < tend) {
      if (regs) {
        float fv[EL];
#pragma unroll
        for (int e = 0; e < EL; ++e) {
          lgv[e] = e < E ? lgv[e] : -INFINITY;
          fv[e] = 0.f;
        }
        if (cf.ca != 0.f) {  // the dispatch fractions (the aux term only)
#pragma unroll
          for (int e = 0; e < EL; ++e) fv[e] = e < E ? (float)cnt[min(e, E - 1)] * cf.inv_nk : 0.f;
        }
        float gkv[KR];
#pragma unroll
        for (int k = 0; k < KR; ++k) gkv[k] = __uint_as_float(gw16 ? gkraw[k] << 16 : gkraw[k]);
        glogit_token_regs<EL, KR>(lgv, fv, ikv, gkv, gw != nullptr, cf, K, gl);
      } else if constexpr (KR != 2) {
        glogit_token<1, EL>(logits, idx, gw, gw_dt, cnt, cf, t, E, K, 0, gl);
      }
    } else {
#pragma unroll
      for (int e = 0; e < EL; ++e) gl[e] = 0.f;
    }
    if (r < nst * 32) {
#pragma unroll
      for (int c8 = 0; c8 < GS; c8 += 8) {
        u32x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e0 = c8 + 2 * j, e1 = e0 + 1;
          const float v0 = (e0 < EL && e0 < E) ? gl[e0 < EL ? e0 : 0] : 0.f;
          const float v1 = (e1 < EL && e1 < E) ? gl[e1 < EL ? e1 : 0] : 0.f;
          w[j] = pack2bf(v0, v1);
        }
        *reinterpret_cast<u32x4*>(&gs[r * GP + c8]) = w;
      }
#pragma unroll
      for (int e = 0; e < NTE * 16; ++e) gts[e * GTP + r] = (e < EL && e < E) ? f2bf(gl[e < EL ? e : 0]) : (uint16_t)0;
      // the first column block of each chunk also hands G (bf16, g_pitch <= 16 expert slots) to the caller
      if (g_out != nullptr && ht == 0 && t < tend) {
        for (int c8 = 0; c8 < g_pitch; c8 += 8)
          *reinterpret_cast<u32x4*>(g_out + (int64_t)t * g_pitch + c8) =
              *reinterpret_cast<const u32x4*>(&gs[r * GP + c8]);
      }
    }
  }

  // gate fragments for dx: B[k = e][n = h] = wg[h][e]
  i16x8 wB[4];
  if (E == 8) {  // each gate row is one 16-byte piece (lanes past the first 8 experts hold zeros)
#pragma unroll
    for (int nc = 0; nc < 4; ++nc) {
      const i16x8 v = *reinterpret_cast<const i16x8*>(wg + (int64_t)(col0 + nc * 16 + n) * 8);
      wB[nc] = g == 0 ? v : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  } else {
#pragma unroll
    for (int nc = 0; nc < 4; ++nc) {
      const int h = col0 + nc * 16 + n;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int e = g * 8 + j;
        wB[nc][j] = (short)wg[(int64_t)h * E + min(e, E - 1)];
        if (e >= E) wB[nc][j] = 0;
      }
    }
  }
  f32x4 accw[4][NTE];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ne = 0; ne < NTE; ++ne) accw[mt][ne] = f32x4{0.f, 0.f, 0.f, 0.f};
  lds_sync();  // G staged

  // One 32-token step.  The refill of r (two steps ahead) is issued as soon as the tile is in LDS and
  // before this step's dx stores: loads and stores retire in order on one counter, so a refill issued
  // after the stores could only be waited for together with them.
  auto step = [&](u32x4(&r)[4], int s) {
    const int lr0 = 32 * s;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = tbeg + lr0 + (lane >> 3) + 8 * j < tend;
      const u32x4 v = r[j];
      *reinterpret_cast<u32x4*>(&xsw[((lane >> 3) + 8 * j) * kSXP + (lane & 7) * 8]) =
          u32x4{ok ? v[0] : 0u, ok ? v[1] : 0u, ok ? v[2] : 0u, ok ? v[3] : 0u};
    }
    // the addend rows of this step's dx, requested before the x refill so that waiting for them at the
    // stores leaves the refill in flight (loads complete in order)
    u32x4 ad[4];
    if (dx_add != nullptr) load_rows(dx_add, ad, tbeg + lr0);
    load_x(r, tbeg + lr0 + 64);
    // dwg: D[m = h][n = e] += sum_t x[t][h] G[t][e]; A from two transposing reads: x[8g .. 8g+7][mt*16 + n]
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int cc = mt * 16 + 4 * (n & 3);
      const sh4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sh4*)&xsw[(8 * g + (n >> 2)) * kSXP + cc]);
      const sh4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sh4*)&xsw[(8 * g + 4 + (n >> 2)) * kSXP + cc]);
      const i16x8 a = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int ne = 0; ne < NTE; ++ne) {
        const i16x8 b = *reinterpret_cast<const i16x8*>(&gts[(ne * 16 + n) * GTP + lr0 + g * 8]);
        accw[mt][ne] = mfma16x16x32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), accw[mt][ne]);
      }
    }
    if (dx == nullptr) return;  // dwg only (the caller forms dx from G itself)
    // dx: D[m = t][n = h] = sum_e G[t][e] wg[h][e], written over the x tile
#pragma unroll
    for (int mk = 0; mk < 2; ++mk) {
      // k = 32 expert slots per MFMA: the slots past GS are zero
      const i16x8 a = g * 8 < GS ? *reinterpret_cast<const i16x8*>(&gs[(lr0 + mk * 16 + n) * GP + g * 8])
                                 : i16x8{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
      for (int nc = 0; nc < 4; ++nc) {
        const f32x4 d = mfma16x16x32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, wB[nc]),
                                     f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int i = 0; i < 4; ++i) xsw[(mk * 16 + g * 4 + i) * kSXP + nc * 16 + n] = f2bf(d[i]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int lr = (lane >> 3) + 8 * j;
      const int t = tbeg + lr0 + lr;
      u32x4 v = *reinterpret_cast<const u32x4*>(&xsw[lr * kSXP + (lane & 7) * 8]);
      if (dx_add != nullptr) v = add_bf16x8(v, ad[j]);
      if (t < tend) *reinterpret_cast<u32x4*>(dx + (int64_t)t * H + col0 + (lane & 7) * 8) = v;
    }
  };

  for (int s = 0; s < nst; s += 2) {
    step(xa, s);
    step(xb, s + 1);
  }

  float* out = ws_dw + (int64_t)chunk * H * E;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ne = 0; ne < NTE; ++ne)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = col0 + mt * 16 + g * 4 + i;
        const int e = ne * 16 + n;
        if (e < E) out[(int64_t)h * E + e] = accw[mt][ne][i];
      }
}

// ---------------------------------------------------------------------------
// Backward 2, wide form (bf16 x bf16, 32 < E <= 128 as EK = 2 or 4 chunks of 32 experts, H % 256 == 0):
// dx = G wg^T and the dwg partial x^T G of one (token chunk, 256 hidden columns) block, with G = dL/dlogits
// in bf16 ([N, EKP], from k_router_glogits).  With many experts the fp32 dwg partials ([chunks, H, E]) are
// as large as x unless the chunks are long, so each block covers ~N * nht / 256 tokens (about one block
// per CU).  Per 32-token step the block stages the step's G rows in LDS (two buffers, one barrier per
// step) and each wave works on its 64 hidden columns: the x tile goes to a wave-private LDS tile, the dwg
// operands x^T (A) and G^T (B) are transposing reads of the x and G tiles, and dx (k = expert) takes G rows
// as A and the gate rows (held in registers for the whole chunk) as B; dx is written back through the x
// tile as 16-byte row segments.  x is prefetched two steps ahead, G one.
// ---------------------------------------------------------------------------
constexpr int kWideBwdBlocks = 256;  // target block count of the wide backward

template <int EK>
constexpr int wide_gpitch() { return EK == 4 ? 128 + 72 : EK * 32 + 8; }  // 36 dwords mod 64 between rows

template <int EK, int NTE>
__global__ __launch_bounds__(256) void k_router_dxdw_wide(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ wg,
                                                          const uint16_t* __restrict__ gb, int N, int H, int E,
                                                          int tc_len, int nht, uint16_t* __restrict__ dx,
                                                          const uint16_t* __restrict__ dx_add,
                                                          float* __restrict__ ws_dw) {
  constexpr int EKP = EK * 32;
  constexpr int GP = wide_gpitch<EK>();  // G tile pitch (bf16): 16-byte rows, conflict-free reads below
  constexpr int GU = EKP / 8;            // 16-byte units per G row
  constexpr int GPT = (32 * GU + 255) / 256;  // G units per thread per step
  __shared__ __attribute__((aligned(16))) uint16_t gs[2][32 * GP];
  __shared__ __attribute__((aligned(16))) uint16_t xs[4][32 * kSXP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 4;
  const int n = lane & 15;
  const int chunk = blockIdx.x / nht;
  const int ht = blockIdx.x - chunk * nht;
  const int tbeg = chunk * tc_len;
  const int tend = min(N, tbeg + tc_len);
  const int nst = ((tend - tbeg + 63) / 64) * 2;  // 32-token steps, rounded up to even
  const int col0 = ht * 256 + wv * 64;            // this wave's first hidden column
  uint16_t* xsw = xs[wv];

  // x stream: lane loads rows (lane/8) + 8j of the step, 16-byte chunk lane%8 of the wave's 64 columns
  // (rows past the chunk re-read its last row and are zeroed when written to LDS)
  const uint16_t* xw = x + col0 + (lane & 7) * 8;
  auto load_x = [&](u32x4(&r)[4], int ts0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = ts0 + (lane >> 3) + 8 * j;
      r[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(xw + (int64_t)min(t, tend - 1) * H));
    }
  };
  // the same rows of an [N, H] bf16 tensor (the dx addend), same clamping
  auto load_rows = [&](const uint16_t* src, u32x4(&r)[4], int ts0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = ts0 + (lane >> 3) + 8 * j;
      r[j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(src + col0 + (lane & 7) * 8 + (int64_t)min(t, tend - 1) * H));
    }
  };
  // G stream: unit q = tid + 256 j of the step is row q / GU, 16-byte unit q % GU
  auto load_g = [&](u32x4(&r)[GPT], int ts0) {
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      const int q = tid + 256 * j;
      const int t = ts0 + q / GU;
      r[j] = q < 32 * GU ? *reinterpret_cast<const u32x4*>(gb + (int64_t)min(t, tend - 1) * EKP + (q % GU) * 8)
                         : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store_g = [&](const u32x4(&r)[GPT], int ts0, uint16_t* gt) {
#pragma unroll
    for (int j = 0; j < GPT; ++j) {
      const int q = tid + 256 * j;
      if (q < 32 * GU) {
        const bool ok = ts0 + q / GU < tend;
        *reinterpret_cast<u32x4*>(&gt[(q / GU) * GP + (q % GU) * 8]) =
            u32x4{ok ? r[j][0] : 0u, ok ? r[j][1] : 0u, ok ? r[j][2] : 0u, ok ? r[j][3] : 0u};
      }
    }
  };
  u32x4 xa[4], xb[4], ga[GPT];
  load_x(xa, tbeg);
  load_x(xb, tbeg + 32);
  load_g(ga, tbeg);

  // gate fragments for dx: B[k = e][n = h] = wg[h][e], e = 32 ek + 8 g + j (zero past E)
  i16x8 wB[4][EK];
#pragma unroll
  for (int nc = 0; nc < 4; ++nc) {
    const uint16_t* wr = wg + (int64_t)(col0 + nc * 16 + n) * E;
#pragma unroll
    for (int ek = 0; ek < EK; ++ek) {
      const int e0 = ek * 32 + g * 8;
      if ((E & 7) == 0 && e0 + 8 <= E) {  // 16-byte aligned row segment
        wB[nc][ek] = *reinterpret_cast<const i16x8*>(wr + e0);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) wB[nc][ek][j] = e0 + j < E ? (short)wr[e0 + j] : (short)0;
      }
    }
  }
  f32x4 accw[4][NTE];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ne = 0; ne < NTE; ++ne) accw[mt][ne] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](u32x4(&r)[4], int s) {
    const int lr0 = 32 * s;
    uint16_t* gt = gs[s & 1];
    store_g(ga, tbeg + lr0, gt);
    if (s + 1 < nst) load_g(ga, tbeg + lr0 + 32);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const bool ok = tbeg + lr0 + (lane >> 3) + 8 * j < tend;
      const u32x4 v = r[j];
      *reinterpret_cast<u32x4*>(&xsw[((lane >> 3) + 8 * j) * kSXP + (lane & 7) * 8]) =
          u32x4{ok ? v[0] : 0u, ok ? v[1] : 0u, ok ? v[2] : 0u, ok ? v[3] : 0u};
    }
    u32x4 ad[4];  // this step's dx addend rows, requested before the x refill (see the streaming form)
    if (dx_add != nullptr) load_rows(dx_add, ad, tbeg + lr0);
    load_x(r, tbeg + lr0 + 64);
    lds_sync();  // the step's G tile is visible to every wave (and every wave is done with step s-1)
    // dwg: D[m = h][n = e] += sum_t x[t][h] G[t][e]; A = x^T and B = G^T from transposing reads
    i16x8 bG[NTE];
#pragma unroll
    for (int ne = 0; ne < NTE; ++ne) {
      const int cc = ne * 16 + 4 * (n & 3);
      const sh4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sh4*)&gt[(8 * g + (n >> 2)) * GP + cc]);
      const sh4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sh4*)&gt[(8 * g + 4 + (n >> 2)) * GP + cc]);
      bG[ne] = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int cc = mt * 16 + 4 * (n & 3);
      const sh4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sh4*)&xsw[(8 * g + (n >> 2)) * kSXP + cc]);
      const sh4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_sh4*)&xsw[(8 * g + 4 + (n >> 2)) * kSXP + cc]);
      const i16x8 a = i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int ne = 0; ne < NTE; ++ne)
        accw[mt][ne] = mfma16x16x32(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, bG[ne]), accw[mt][ne]);
    }
    if (dx == nullptr) return;  // dwg only (the caller forms dx from G itself)
    // dx: D[m = t][n = h] = sum_e G[t][e] wg[h][e], written over the x tile
#pragma unroll
    for (int mk = 0; mk < 2; ++mk) {
      i16x8 aG[EK];
#pragma unroll
      for (int ek = 0; ek < EK; ++ek) aG[ek] = *reinterpret_cast<const i16x8*>(&gt[(mk * 16 + n) * GP + ek * 32 + g * 8]);
#pragma unroll
      for (int nc = 0; nc < 4; ++nc) {
        f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ek = 0; ek < EK; ++ek)
          d = mfma16x16x32(__builtin_bit_cast(bf16x8, aG[ek]), __builtin_bit_cast(bf16x8, wB[nc][ek]), d);
#pragma unroll
        for (int i = 0; i < 4; ++i) xsw[(mk * 16 + g * 4 + i) * kSXP + nc * 16 + n] = f2bf(d[i]);
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int lr = (lane >> 3) + 8 * j;
      const int t = tbeg + lr0 + lr;
      u32x4 v = *reinterpret_cast<const u32x4*>(&xsw[lr * kSXP + (lane & 7) * 8]);
      if (dx_add != nullptr) v = add_bf16x8(v, ad[j]);
      if (t < tend)
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(dx + (int64_t)t * H + col0 + (lane & 7) * 8));
    }
  };

  for (int s = 0; s < nst; s += 2) {
    step(xa, s);
    step(xb, s + 1);
  }

  float* out = ws_dw + (int64_t)chunk * H * E;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int ne = 0; ne < NTE; ++ne)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = col0 + mt * 16 + g * 4 + i;
        const int e = ne * 16 + n;
        if (e < E) out[(int64_t)h * E + e] = accw[mt][ne][i];
      }
}

// Backward, fp32 x and gate (E <= 16, H % 4 == 0, x and dx 16-byte aligned): dx = G wg^T and the per-chunk
// partials of dwg = x^T G in one pass over x.  Block = 4 waves on one 256-column slice of the hidden dim
// (blockIdx.x) and one chunk of tc_len tokens (blockIdx.y); lane l owns columns h = h0 + 4 l .. h + 3 and keeps
// their gate rows in registers.  Wave w takes the chunk's tokens w, w + 4, ...: per token it reads the row G[t]
// (wave-uniform), its 4 x values (one 16-byte load), stores its 4 dx values (one 16-byte store: each a sum
// over e = 0 .. E-1 in order) and adds x * G into its 4 x EL dwg sums.  The 4 waves' sums are added in wave
// order through LDS and stored as the chunk's partial ws_dw[chunk][h * E + e] (the fixed-order reduce over
// chunks follows).
template <int EL>
__global__ __launch_bounds__(256) void k_router_dxdw_f32(const float* __restrict__ x, const float* __restrict__ wg,
                                                         const float* __restrict__ G, int N, int H, int E,
                                                         int tc_len, float* __restrict__ dx,
                                                         float* __restrict__ ws_dw) {
  __shared__ float s_part[3][4 * EL][65];  // waves 1-3's sums, [wave][i * EL + e][lane] (padded rows)
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int h = blockIdx.x * 256 + 4 * lane;
  const bool hv = h < H;
  const int tbeg = blockIdx.y * tc_len;
  const int tend = min(N, tbeg + tc_len);
  float gr[4][EL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < EL; ++e) gr[i][e] = (hv && e < E) ? wg[(int64_t)(h + i) * E + e] : 0.f;
  float acc[4][EL];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int e = 0; e < EL; ++e) acc[i][e] = 0.f;
#pragma unroll 2
  for (int t = tbeg + wv; t < tend; t += 4) {
    float g[EL];
#pragma unroll
    for (int e = 0; e < EL; ++e) g[e] = e < E ? G[(int64_t)t * E + e] : 0.f;
    const f32x4 xv = hv ? __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(x + (int64_t)t * H + h))
                        : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = 0.f;
#pragma unroll
      for (int e = 0; e < EL; ++e) v = fmaf(g[e], gr[i][e], v);
      o[i] = v;
    }
    if (hv) __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(dx + (int64_t)t * H + h));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < EL; ++e) acc[i][e] = fmaf(xv[i], g[e], acc[i][e]);
  }
  if (wv > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < EL; ++e) s_part[wv - 1][i * EL + e][lane] = acc[i][e];
  }
  __syncthreads();
  if (wv == 0 && hv) {
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < EL; ++e) acc[i][e] += s_part[w][i * EL + e][lane];
    float* dst = ws_dw + (int64_t)blockIdx.y * H * E + (int64_t)h * E;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < EL; ++e)
        if (e < E) dst[i * E + e] = acc[i][e];
  }
}

// Generic dx = G wg^T: one thread per (t, h).
__global__ __launch_bounds__(256) void k_router_dx_generic(const float* __restrict__ G, const void* __restrict__ wg,
                                                           int w_dt, int N, int H, int E, void* __restrict__ dx,
                                                           int x_dt) {
  const int64_t total = (int64_t)N * H;
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < total; q += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = q / H;
    const int h = (int)(q % H);
    float acc = 0.f;
    for (int e = 0; e < E; ++e) acc = fmaf(G[t * E + e], load_f(wg, w_dt, (int64_t)h * E + e), acc);
    store_f(dx, x_dt, q, acc);
  }
}

// Generic dwg partial per token chunk: thread per (h, e).
__global__ __launch_bounds__(256) void k_router_dw_generic(const void* __restrict__ x, int x_dt,
                                                           const float* __restrict__ G, int N, int H, int E,
                                                           int tc_len, float* __restrict__ ws_dw) {
  const int64_t he = (int64_t)H * E;
  const int tbeg = blockIdx.y * tc_len;
  const int tend = min(N, tbeg + tc_len);
  for (int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; q < he; q += (int64_t)gridDim.x * blockDim.x) {
    const int h = (int)(q / E);
    const int e = (int)(q % E);
    float acc = 0.f;
    for (int t = tbeg; t < tend; ++t) acc = fmaf(load_f(x, x_dt, (int64_t)t * H + h), G[(int64_t)t * E + e], acc);
    ws_dw[(int64_t)blockIdx.y * he + q] = acc;
  }
}

// out = sum over token chunks of ws[c][*], fixed order.  A block covers 64
// groups of VEC consecutive outputs; its 4 waves sum interleaved chunk
// subsets, then wave 0 adds the 4 partials in order.
template <int VEC>
__global__ __launch_bounds__(256) void k_reduce_chunks(const float* __restrict__ ws, int nchunk, int64_t len,
                                                       void* __restrict__ out, int out_dt) {
  __shared__ float s[4][64][VEC];
  const int qi = threadIdx.x & 63;
  const int cg = threadIdx.x >> 6;
  const int64_t ngroups = len / VEC;
  for (int64_t gb = (int64_t)blockIdx.x * 64; gb < ngroups; gb += (int64_t)gridDim.x * 64) {
    const int64_t q = gb + qi;
    float a[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) a[v] = 0.f;
    if (q < ngroups && ws != nullptr) {
      // chunks cg, cg+4, ... summed in that order; loaded 8 at a time so the loads overlap
      int c = cg;
      for (; c + 28 < nchunk; c += 32) {
        float xv[8][VEC];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const float* src = ws + (int64_t)(c + 4 * u) * len + q * VEC;
          if constexpr (VEC == 4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
            for (int v = 0; v < 4; ++v) xv[u][v] = x[v];
          } else {
#pragma unroll
            for (int v = 0; v < VEC; ++v) xv[u][v] = src[v];
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int v = 0; v < VEC; ++v) a[v] += xv[u][v];
      }
      for (; c < nchunk; c += 4) {
        const float* src = ws + (int64_t)c * len + q * VEC;
#pragma unroll
        for (int v = 0; v < VEC; ++v) a[v] += src[v];
      }
    }
#pragma unroll
    for (int v = 0; v < VEC; ++v) s[cg][qi][v] = a[v];
    __syncthreads();
    if (cg == 0 && q < ngroups) {
#pragma unroll
      for (int v = 0; v < VEC; ++v)
        store_f(out, out_dt, q * VEC + v, ((s[0][qi][v] + s[1][qi][v]) + s[2][qi][v]) + s[3][qi][v]);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

// Hidden-dim split (HS) and prefetch depth (U) of the forward kernel per expert-tile count.
constexpr int fwd_hs(int NT) { return NT == 1 ? 4 : (NT == 2 ? 2 : 1); }
constexpr int fwd_u(int NT) { return NT <= 4 ? 4 : 2; }
int fwd_tokens_per_block(int NT) { return 16 * (4 / fwd_hs(NT)); }

struct FwdPlan {
  bool f32;     // k_router_fwd_f32 (fp32 x and gate, E <= 64, H % 4 == 0)
  bool mfma;
  bool stream;  // k_router_fwd_stream (E <= 32, H % 256 == 0)
  bool wide;    // k_router_fwd_wide (32 < E <= 256, H % 64 == 0)
  int NT, TG;
  int nblk;
  size_t off_wp, off_cnt, off_p, off_z, off_ticket, total;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

FwdPlan plan_fwd(int64_t N, int64_t H, int64_t E, int x_dt, int w_dt, bool allow_stream = true) {
  FwdPlan p{};
  p.mfma = x_dt == MOE_BF16 && w_dt == MOE_BF16 && H % 32 == 0 && E <= 128;
  p.NT = (int)((E + 15) / 16);
  if (p.NT == 3) p.NT = 4;
  if (p.NT > 4 && p.NT < 8) p.NT = 8;
  p.stream = allow_stream && p.mfma && E <= 32 && H % 256 == 0;
  p.wide = allow_stream && x_dt == MOE_BF16 && w_dt == MOE_BF16 && E > 32 && E <= kMaxE && H % 64 == 0;
  p.f32 = allow_stream && x_dt == MOE_F32 && w_dt == MOE_F32 && E <= 64 && H % 4 == 0;
  if (p.f32) {
    // 16 * TG tokens per block: the largest TG that still gives about one block per CU (256)
    const int64_t groups = cdiv(N, 16);
    p.TG = groups >= 256 * 8 ? 8 : (groups >= 256 * 4 ? 4 : (groups >= 256 * 2 ? 2 : 1));
    p.nblk = cdiv(N, 16 * p.TG);
  } else if (p.wide) {
    p.mfma = true;
    p.NT = E <= 64 ? 4 : (E <= 128 ? 8 : 16);
    p.nblk = cdiv(N, WideFwd<4>::ROWS);
  } else if (p.stream) {
    // 16 * TG tokens per block: the largest TG that still gives one block per CU (256)
    p.TG = N >= 256 * 64 ? 4 : (N >= 256 * 32 ? 2 : 1);
    p.nblk = cdiv(N, 16 * p.TG);
  } else if (p.mfma) {
    p.nblk = cdiv(N, fwd_tokens_per_block(p.NT));
  } else {
    p.nblk = (int)std::min<int64_t>(512, std::max<int64_t>(1, (N + 15) / 16));
  }
  // the ticket word sits at offset 0 in every layout: calls that reuse one workspace with different
  // shapes or paths never write over it, and each streaming call leaves it at zero
  size_t off = 0;
  p.off_ticket = off;
  off += 256;
  p.off_wp = off;
  off += p.mfma ? align256((size_t)((H + 31) / 32) * p.NT * 64 * 16) : 0;
  p.off_cnt = off;
  off += align256((size_t)p.nblk * E * sizeof(int));
  p.off_p = off;
  off += align256((size_t)p.nblk * E * sizeof(float));
  p.off_z = off;
  off += align256((size_t)p.nblk * 2 * sizeof(float));
  p.total = off;
  return p;
}

struct BwdPlan {
  bool f32;     // k_router_glogits + k_router_dxdw_f32 (fp32 x and gate, E <= 16, H % 4 == 0)
  bool mfma;
  bool stream;  // k_router_dxdw_stream (E <= 32, H % 256 == 0)
  bool wide;    // k_router_glogits + k_router_dxdw_wide (32 < E <= 128, H % 256 == 0)
  int EK, NTE;
  int nchunk, tc_len;
  size_t off_g, off_gb, off_ws, total;
};

BwdPlan plan_bwd(int64_t N, int64_t H, int64_t E, int x_dt, int w_dt) {
  BwdPlan p{};
  p.mfma = x_dt == MOE_BF16 && w_dt == MOE_BF16 && H % 64 == 0 && E <= 128;
  p.EK = (int)((E + 31) / 32);
  if (p.EK == 3) p.EK = 4;
  p.NTE = (int)((E + 15) / 16);
  if (p.NTE == 3) p.NTE = 4;
  if (p.NTE > 4 && p.NTE < 8) p.NTE = 8;
  p.stream = p.mfma && E <= 32 && H % 256 == 0;
  p.wide = p.mfma && E > 32 && H % 256 == 0;
  p.f32 = x_dt == MOE_F32 && w_dt == MOE_F32 && E <= 16 && H % 4 == 0;
  if (p.f32) {
    // about 1024 blocks of (256-column slice, token chunk), at most 8 tokens per wave before the chunks grow
    const int64_t nht = cdiv(H, 256);
    const int64_t want = std::max<int64_t>(1, 1024 / nht);
    p.nchunk = (int)std::max<int64_t>(1, std::min<int64_t>(want, cdiv(N, 32)));
    p.tc_len = (int)cdiv(N, p.nchunk);
    p.nchunk = (int)cdiv(N, p.tc_len);
  } else if (p.wide) {
    // about one block per CU; long chunks keep the fp32 dwg partials few
    const int nht = (int)(H / 256);
    const int want = std::max(1, kWideBwdBlocks / nht);
    p.tc_len = std::max(64, cdiv(cdiv(N, want), 64) * 64);
    p.nchunk = cdiv(N, p.tc_len);
  } else if (p.stream) {
    // one round of blocks: per CU four 4-wave blocks (or one 16-wave block with E <= 8 and H % 1024 == 0)
    // with up to 16 experts (at most 128 registers), two 4-wave blocks with more (the second expert tile's
    // registers); chunks of a multiple of 64 tokens, at most kSTC
    const int nht = (int)(H / 256);
    const int want = std::max(1, (E <= 16 ? 1024 : 512) / nht);
    p.tc_len = std::min(kSTC, std::max(64, cdiv(cdiv(N, want), 64) * 64));
    p.nchunk = cdiv(N, p.tc_len);
  } else if (p.mfma) {
    const int nhb = cdiv(H, 256);
    int nchunk = std::max(1, 1024 / nhb);
    const int max_chunks = cdiv(N, kBwdTS);
    nchunk = std::min(nchunk, max_chunks);
    p.tc_len = cdiv(cdiv(N, nchunk), kBwdTS) * kBwdTS;
    p.nchunk = cdiv(N, p.tc_len);
  } else {
    p.tc_len = 256;
    p.nchunk = cdiv(N, p.tc_len);
  }
  if (p.nchunk < 1) p.nchunk = 1;
  size_t off = 0;
  p.off_g = off;  // G (and its bf16 copy) for the non-streaming paths, which an unaligned call falls back to
  off += align256((size_t)N * E * sizeof(float));
  p.off_gb = off;
  off += p.mfma ? align256((size_t)N * p.EK * 32 * sizeof(uint16_t)) : 0;
  p.off_ws = off;
  off += align256((size_t)p.nchunk * H * E * sizeof(float));
  p.total = off;
  return p;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// dx += dx_add element-wise (same dtype; a bf16 sum is formed in fp32 and rounded once, as a tensor addition
// is), for the backward forms that do not fold the addend into their dx stores.
__global__ __launch_bounds__(256) void k_add_rows(void* __restrict__ dx, const void* __restrict__ add, int64_t n,
                                                  int dt) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride)
    store_f(dx, dt, i, load_f(dx, dt, i) + load_f(add, dt, i));
}

void launch_add_rows(hipStream_t s, void* dx, const void* add, int64_t n, int dt) {
  MOE_LAUNCH("k_add_rows", k_add_rows, dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>(16384, (n + 255) / 256))),
             dim3(256), 0, s, dx, add, n, dt);
}

void launch_reduce(hipStream_t s, const float* ws, int nchunk, int64_t len, void* out, int out_dt) {
  if (len % 4 == 0) {
    const unsigned nb = (unsigned)std::max<int64_t>(1, std::min<int64_t>(2048, (len / 4 + 63) / 64));
    MOE_LAUNCH("k_reduce_chunks", k_reduce_chunks<4>, dim3(nb), dim3(256), 0, s, ws, nchunk, len, out, out_dt);
  } else {
    const unsigned nb = (unsigned)std::max<int64_t>(1, std::min<int64_t>(2048, (len + 63) / 64));
    MOE_LAUNCH("k_reduce_chunks", k_reduce_chunks<1>, dim3(nb), dim3(256), 0, s, ws, nchunk, len, out, out_dt);
  }
}

template <int NT, int TG>
void launch_fwd_stream(int nblk, hipStream_t s, const uint16_t* x, const uint16_t* wg, const float* bias, int N, int H,
                       int E, int K, int64_t* idx, void* w, int w_dt, float* logits, float* lse, int* pc, float* pp,
                       float* pz, unsigned* ticket, float aux_coef, float z_coef, int64_t* cnt, float* stats,
                       float* aux_out, float* z_out) {
  MOE_LAUNCH("k_router_fwd_bf16", (k_router_fwd_stream<NT, TG>), dim3(nblk), dim3(512), 0, s, x, wg, bias, N, H, E, K,
             idx, w, w_dt, logits, lse, pc, pp, pz, ticket, aux_coef, z_coef, cnt, stats, aux_out, z_out);
}

template <int NT>
void launch_fwd_mfma(dim3 grid, hipStream_t s, const uint16_t* x, const i16x8* wp, const float* bias, int N, int H,
                     int E, int K, int64_t* idx, void* w, int w_dt, float* logits, float* lse, int* pc, float* pp,
                     float* pz) {
  constexpr int HS = fwd_hs(NT);
  constexpr int U = fwd_u(NT);
  MOE_LAUNCH("k_router_fwd_bf16", (k_router_fwd_bf16<NT, HS, U>), grid, dim3(256), 0, s, x, wp, bias, N, H, E, K, idx, w, w_dt,
                     logits, lse, pc, pp, pz);
}

template <int NTE>
void launch_dxdw_stream(hipStream_t s, const uint16_t* x, const uint16_t* wg, const float* logits, const int64_t* idx,
                        const void* gw, int gw_dt, const int64_t* cnt, const float* grad_aux, const float* grad_z,
                        float aux_coef, float z_coef, int N, int H, int E, int K, int tc_len, int nchunk, uint16_t* dx,
                        float* ws, uint16_t* g_out = nullptr, int g_pitch = 0, const uint16_t* dx_add = nullptr) {
  const char* name = dx ? "k_router_dxdw_bf16" : "k_router_dw_bf16";
#define MOE_DXDW_STREAM(EL_, KR_, WPB_)                                                                               \
  MOE_LAUNCH(name, (k_router_dxdw_stream<NTE, EL_, KR_, WPB_>), dim3((unsigned)(nchunk * (H / (64 * WPB_)))),          \
             dim3(64 * WPB_), 0, s, x, wg, logits, idx, gw, gw_dt, cnt, grad_aux, grad_z, aux_coef, z_coef, N, H, E, K,  \
             tc_len, H / (64 * WPB_), dx, dx_add, ws, g_out, g_pitch)
  // G over 8 expert slots when E <= 8 (fewer registers while the first x tiles are in flight); the top-k
  // slots preloaded: 2 when K <= 2 (shorter code: the prologue runs on a cold instruction cache), else 4;
  // 16-wave blocks (1024 columns) when H allows
  if constexpr (NTE == 1) {
    if (E <= 8) {
      if (H % 1024 == 0) {
        if (K <= 2) MOE_DXDW_STREAM(8, 2, 16);
        else MOE_DXDW_STREAM(8, kGRegK, 16);
      } else {
        if (K <= 2) MOE_DXDW_STREAM(8, 2, 4);
        else MOE_DXDW_STREAM(8, kGRegK, 4);
      }
      return;
    }
  }
  if (K <= 2) MOE_DXDW_STREAM(NTE * 16, 2, 4);
  else MOE_DXDW_STREAM(NTE * 16, kGRegK, 4);
#undef MOE_DXDW_STREAM
}

template <int EK, int NTE>
void launch_dxdw(dim3 grid, hipStream_t s, const uint16_t* x, const uint16_t* wg, const uint16_t* gb, int N, int H,
                 int E, int tc_len, uint16_t* dx, float* ws) {
  MOE_LAUNCH("k_router_dxdw_bf16", (k_router_dxdw_bf16<EK, NTE>), grid, dim3(256), 0, s, x, wg, gb, N, H, E, tc_len, dx, ws);
}

}  // namespace

bool router_dw_g_applies(int64_t H, int64_t E) { return E <= 16 && H % 256 == 0; }

size_t router_dw_g_workspace(int64_t N, int64_t H, int64_t E) {
  const BwdPlan p = plan_bwd(N > 0 ? N : 1, H, E, MOE_BF16, MOE_BF16);
  return align256((size_t)p.nchunk * H * E * sizeof(float));
}

int router_dw_g(const uint16_t* x, const uint16_t* wg, const float* logits, const int64_t* idx, const void* grad_w,
                int gw_dtype, const int64_t* cnt, const float* grad_aux, const float* grad_z, float aux_coef,
                float z_coef, int64_t N, int64_t H, int64_t E, int64_t K, void* dwg_out, uint16_t* g_out, int g_pitch,
                void* ws, hipStream_t s) {
  const BwdPlan p = plan_bwd(N, H, E, MOE_BF16, MOE_BF16);
  float* wsdw = static_cast<float*>(ws);
  launch_dxdw_stream<1>(s, x, wg, logits, idx, grad_w, gw_dtype, cnt, grad_aux, grad_z, aux_coef, z_coef, (int)N,
                        (int)H, (int)E, (int)K, p.tc_len, p.nchunk, nullptr, wsdw, g_out, g_pitch);
  if (int rc = check_launch("k_router_dw_bf16")) return rc;
  launch_reduce(s, wsdw, p.nchunk, H * E, dwg_out, MOE_BF16);
  return check_launch("router_dw_g");
}

}  // namespace moe

using namespace moe;

extern "C" size_t moe_router_fwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype, int wg_dtype) {
  (void)K;
  if (N <= 0 || H <= 0 || E <= 0) return 0;
  return std::max(plan_fwd(N, H, E, x_dtype, wg_dtype).total, plan_fwd(N, H, E, x_dtype, wg_dtype, false).total);
}

extern "C" int64_t moe_router_fwd_lds_bytes(int64_t N, int64_t H, int64_t E, int x_dtype, int wg_dtype) {
  if (N <= 0 || H <= 0 || E < 1 || E > kMaxE) return 0;
  const FwdPlan p = plan_fwd(N, H, E, x_dtype, wg_dtype);
  const void* f = nullptr;
  if (p.f32) {
    // the MFMA form when x is 16-byte aligned (the usual case); all TG variants share their LDS layout per NT
    f = p.NT == 1 ? (const void*)k_router_fwd_f32<1, 1> : p.NT == 2 ? (const void*)k_router_fwd_f32<2, 1>
                                                                     : (const void*)k_router_fwd_f32<4, 1>;
  } else if (p.wide) {
    f = p.NT == 4 ? (const void*)k_router_fwd_wide<4> : p.NT == 8 ? (const void*)k_router_fwd_wide<8>
                                                                 : (const void*)k_router_fwd_wide<16>;
  } else if (p.stream) {
    if (p.NT == 1) f = p.TG == 4 ? (const void*)k_router_fwd_stream<1, 4> : p.TG == 2 ? (const void*)k_router_fwd_stream<1, 2>
                                                                                    : (const void*)k_router_fwd_stream<1, 1>;
    else f = p.TG == 4 ? (const void*)k_router_fwd_stream<2, 4> : p.TG == 2 ? (const void*)k_router_fwd_stream<2, 2>
                                                                           : (const void*)k_router_fwd_stream<2, 1>;
  } else if (p.mfma) {
    switch (p.NT) {
      case 1: f = (const void*)k_router_fwd_bf16<1, fwd_hs(1), fwd_u(1)>; break;
      case 2: f = (const void*)k_router_fwd_bf16<2, fwd_hs(2), fwd_u(2)>; break;
      case 4: f = (const void*)k_router_fwd_bf16<4, fwd_hs(4), fwd_u(4)>; break;
      default: f = (const void*)k_router_fwd_bf16<8, fwd_hs(8), fwd_u(8)>; break;
    }
  } else {
    f = (const void*)k_route_from_logits;
  }
  hipFuncAttributes attr{};
  if (hipFuncGetAttributes(&attr, f) != hipSuccess) {
    (void)hipGetLastError();
    return -1;
  }
  return (int64_t)attr.sharedSizeBytes;
}

extern "C" int moe_router_fwd(const void* x, int x_dtype, const void* wg, int wg_dtype, const float* bias, int64_t N,
                              int64_t H, int64_t E, int64_t K, int64_t* idx_out, void* w_out, int w_dtype,
                              float* logits_out, float* lse_out, int64_t* cnt_out, float* stats_out,
                              float aux_coef, float z_coef, float* aux_out, float* z_out, void* workspace,
                              size_t ws_bytes, void* stream) {
  if (N < 0 || H <= 0 || E < 1 || E > kMaxE || K < 1 || K > E || K > kMaxK)
    return fail_arg("moe_router_fwd: bad shape N=%lld H=%lld E=%lld K=%lld (need 1<=K<=min(E,32), E<=256)",
                    (long long)N, (long long)H, (long long)E, (long long)K);
  if (N > INT32_MAX / 2 || H > INT32_MAX / 2) return fail_arg("moe_router_fwd: N or H too large");
  if ((x_dtype != MOE_F32 && x_dtype != MOE_BF16) || (wg_dtype != MOE_F32 && wg_dtype != MOE_BF16) ||
      (w_dtype != MOE_F32 && w_dtype != MOE_BF16))
    return fail_arg("moe_router_fwd: unsupported dtype");
  if (N == 0) return 0;
  if (!x || !wg || !idx_out || !w_out || !logits_out || !lse_out || !cnt_out || !stats_out)
    return fail_arg("moe_router_fwd: null pointer argument");
  // the streaming form DMAs the gate rows too, so it needs both operands 16-byte aligned
  const FwdPlan p = plan_fwd(N, H, E, x_dtype, wg_dtype, aligned16(x) && aligned16(wg));
  if (ws_bytes < p.total || (!workspace && p.total))
    return set_error("moe_router_fwd: workspace %zu < %zu bytes", ws_bytes, p.total), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int* pc = reinterpret_cast<int*>(ws + p.off_cnt);
  float* pp = reinterpret_cast<float*>(ws + p.off_p);
  float* pz = reinterpret_cast<float*>(ws + p.off_z);
  if (p.f32 && aligned16(x)) {
    // fp32 form: MFMA gate GEMM, routing and the statistics fold in one launch (ticket zero on entry and exit)
    unsigned* ticket = reinterpret_cast<unsigned*>(ws + p.off_ticket);
    const float* xf = static_cast<const float*>(x);
    const float* wf = static_cast<const float*>(wg);
#define MOE_FWDF(NTv, TGv)                                                                                         \
  MOE_LAUNCH("k_router_fwd_f32", (k_router_fwd_f32<NTv, TGv>), dim3(p.nblk), dim3(512), 0, s, xf, wf, bias, (int)N,   \
             (int)H, (int)E, (int)K, idx_out, w_out, w_dtype, logits_out, lse_out, pc, pp, pz, ticket, aux_coef,    \
             z_coef, cnt_out, stats_out, aux_out, z_out)
#define MOE_FWDF_TG(NTv)          \
  do {                            \
    if (p.TG == 8) MOE_FWDF(NTv, 8); \
    else if (p.TG == 4) MOE_FWDF(NTv, 4); \
    else if (p.TG == 2) MOE_FWDF(NTv, 2); \
    else MOE_FWDF(NTv, 1);        \
  } while (0)
    if (p.NT == 1) MOE_FWDF_TG(1);
    else if (p.NT == 2) MOE_FWDF_TG(2);
    else MOE_FWDF_TG(4);
#undef MOE_FWDF_TG
#undef MOE_FWDF
    return check_launch("k_router_fwd_f32");
  }
  const bool mfma = p.mfma && aligned16(x);
  if (mfma && p.stream) {
    // streaming form: raw gate, finalize folded into the last block (ticket zero on entry and on exit)
    unsigned* ticket = reinterpret_cast<unsigned*>(ws + p.off_ticket);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const uint16_t* wb = static_cast<const uint16_t*>(wg);
#define MOE_FWDS(NTv, TGv)                                                                                        \
  launch_fwd_stream<NTv, TGv>(p.nblk, s, xb, wb, bias, (int)N, (int)H, (int)E, (int)K, idx_out, w_out, w_dtype,  \
                              logits_out, lse_out, pc, pp, pz, ticket, aux_coef, z_coef, cnt_out, stats_out, aux_out, \
                              z_out)
    if (p.NT == 1) {
      if (p.TG == 4) MOE_FWDS(1, 4);
      else if (p.TG == 2) MOE_FWDS(1, 2);
      else MOE_FWDS(1, 1);
    } else {
      if (p.TG == 4) MOE_FWDS(2, 4);
      else if (p.TG == 2) MOE_FWDS(2, 2);
      else MOE_FWDS(2, 1);
    }
#undef MOE_FWDS
    return check_launch("k_router_fwd_bf16");
  }
  if (mfma && p.wide) {
    // wide streaming form: packed gate, finalize folded into the last block (ticket zero on entry and on exit)
    i16x8* wp = reinterpret_cast<i16x8*>(ws + p.off_wp);
    const int64_t lanes = (int64_t)(H / 32) * p.NT * 64;
    MOE_LAUNCH("k_pack_gate", k_pack_gate, dim3((unsigned)std::min<int64_t>(1024, (lanes + 255) / 256)), dim3(256), 0, s,
               static_cast<const uint16_t*>(wg), (int)H, (int)E, p.NT, wp, nullptr);
    unsigned* ticket = reinterpret_cast<unsigned*>(ws + p.off_ticket);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
#define MOE_FWDW(NTv)                                                                                               \
  MOE_LAUNCH("k_router_fwd_bf16", (k_router_fwd_wide<NTv>), dim3(p.nblk), dim3(512), 0, s, xb, wp, bias, (int)N,     \
             (int)H, (int)E, (int)K, idx_out, w_out, w_dtype, logits_out, lse_out, pc, pp, pz, ticket, aux_coef,   \
             z_coef, cnt_out, stats_out, aux_out, z_out)
    if (p.NT == 4) MOE_FWDW(4);
    else if (p.NT == 8) MOE_FWDW(8);
    else MOE_FWDW(16);
#undef MOE_FWDW
    return check_launch("k_router_fwd_bf16");
  }
  if (mfma) {
    i16x8* wp = reinterpret_cast<i16x8*>(ws + p.off_wp);
    const int64_t lanes = (int64_t)((H + 31) / 32) * p.NT * 64;
    MOE_LAUNCH("k_pack_gate", k_pack_gate, dim3((unsigned)std::min<int64_t>(1024, (lanes + 255) / 256)), dim3(256), 0, s,
                       static_cast<const uint16_t*>(wg), (int)H, (int)E, p.NT, wp, nullptr);
    const dim3 grid(p.nblk);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    switch (p.NT) {
      case 1: launch_fwd_mfma<1>(grid, s, xb, wp, bias, (int)N, (int)H, (int)E, (int)K, idx_out, w_out, w_dtype, logits_out, lse_out, pc, pp, pz); break;
      case 2: launch_fwd_mfma<2>(grid, s, xb, wp, bias, (int)N, (int)H, (int)E, (int)K, idx_out, w_out, w_dtype, logits_out, lse_out, pc, pp, pz); break;
      case 4: launch_fwd_mfma<4>(grid, s, xb, wp, bias, (int)N, (int)H, (int)E, (int)K, idx_out, w_out, w_dtype, logits_out, lse_out, pc, pp, pz); break;
      case 8: launch_fwd_mfma<8>(grid, s, xb, wp, bias, (int)N, (int)H, (int)E, (int)K, idx_out, w_out, w_dtype, logits_out, lse_out, pc, pp, pz); break;
      default: return fail_arg("moe_router_fwd: internal tile error");
    }
    if (int rc = check_launch("k_router_fwd_bf16")) return rc;
    MOE_LAUNCH("k_router_finalize", k_router_finalize, dim3(1), dim3(kFinThreads), 0, s, pc, pp, pz, p.nblk, (int)N, (int)E, (int)K,
                       aux_coef, z_coef, cnt_out, stats_out, aux_out, z_out);
  } else {
    FwdPlan pg = p;
    if (p.mfma) {  // unaligned x: generic path needs its own block count
      pg = plan_fwd(N, H, E, MOE_F32, MOE_F32);
      if (ws_bytes < pg.total) return set_error("moe_router_fwd: workspace too small"), MOE_EWORKSPACE;
      pc = reinterpret_cast<int*>(ws + pg.off_cnt);
      pp = reinterpret_cast<float*>(ws + pg.off_p);
      pz = reinterpret_cast<float*>(ws + pg.off_z);
    }
    const unsigned lg_blocks = (unsigned)std::min<int64_t>(4096, (N + 3) / 4);
    MOE_LAUNCH("k_logits_generic", k_logits_generic, dim3(lg_blocks), dim3(256), 0, s, x, x_dtype, wg, wg_dtype, bias, (int)N,
                       (int)H, (int)E, logits_out);
    const int tpb = cdiv(N, pg.nblk);
    const int nblk = cdiv(N, tpb);
    MOE_LAUNCH("k_route_from_logits", k_route_from_logits, dim3(nblk), dim3(256), 0, s, logits_out, (int)N, (int)E, (int)K, tpb,
                       idx_out, w_out, w_dtype, lse_out, pc, pp, pz);
    MOE_LAUNCH("k_router_finalize", k_router_finalize, dim3(1), dim3(kFinThreads), 0, s, pc, pp, pz, nblk, (int)N, (int)E, (int)K,
                       aux_coef, z_coef, cnt_out, stats_out, aux_out, z_out);
  }
  return check_launch("moe_router_fwd");
}

extern "C" size_t moe_router_bwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype, int wg_dtype) {
  (void)K;
  if (N <= 0 || H <= 0 || E <= 0) return 0;
  return plan_bwd(N, H, E, x_dtype, wg_dtype).total;
}

extern "C" int moe_router_bwd_acc(const void* x, int x_dtype, const void* wg, int wg_dtype, const float* logits,
                                  const int64_t* idx, const void* grad_w, int gw_dtype, const int64_t* cnt,
                                  const float* grad_aux, const float* grad_z, float aux_coef, float z_coef, int64_t N,
                                  int64_t H, int64_t E, int64_t K, const void* dx_add, void* dx_out, void* dwg_out,
                                  void* workspace, size_t ws_bytes, void* stream) {
  if (N < 0 || H <= 0 || E < 1 || E > kMaxE || K < 1 || K > E)
    return fail_arg("moe_router_bwd: bad shape N=%lld H=%lld E=%lld K=%lld", (long long)N, (long long)H,
                    (long long)E, (long long)K);
  if ((x_dtype != MOE_F32 && x_dtype != MOE_BF16) || (wg_dtype != MOE_F32 && wg_dtype != MOE_BF16) ||
      (gw_dtype != MOE_F32 && gw_dtype != MOE_BF16))
    return fail_arg("moe_router_bwd: unsupported dtype");
  if (!x || !wg || !logits || !idx || !dx_out || !dwg_out) return fail_arg("moe_router_bwd: null pointer argument");
  if (dx_add != nullptr && N > 0) {
    // the addend is read while dx is written: the two must not overlap
    const int64_t nb = N * H * (x_dtype == MOE_BF16 ? 2 : 4);
    const char* a = static_cast<const char*>(dx_add);
    const char* d = static_cast<const char*>(dx_out);
    if (a < d + nb && d < a + nb) return fail_arg("moe_router_bwd: dx_add overlaps dx_out");
  }
  if (aux_coef != 0.f && !cnt) return fail_arg("moe_router_bwd: aux_coef != 0 needs cnt");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const BwdPlan p = plan_bwd(N > 0 ? N : 1, H, E, x_dtype, wg_dtype);
  if (N == 0) {
    const int64_t len = H * E;
    // dwg = 0 when there are no tokens
    launch_reduce(s,
                       static_cast<const float*>(nullptr), 0, len, dwg_out, wg_dtype);
    return check_launch("moe_router_bwd");
  }
  if (ws_bytes < p.total || !workspace)
    return set_error("moe_router_bwd: workspace %zu < %zu bytes", ws_bytes, p.total), MOE_EWORKSPACE;
  char* ws = static_cast<char*>(workspace);
  float* G = reinterpret_cast<float*>(ws + p.off_g);
  float* wsdw = reinterpret_cast<float*>(ws + p.off_ws);
  const bool mfma = p.mfma && aligned16(x) && aligned16(dx_out);
  uint16_t* gb = mfma ? reinterpret_cast<uint16_t*>(ws + p.off_gb) : nullptr;
  int nchunk = p.nchunk;
  const bool add_fused = dx_add != nullptr && x_dtype == MOE_BF16 && aligned16(dx_add);
  const uint16_t* addb = add_fused ? static_cast<const uint16_t*>(dx_add) : nullptr;
  if (mfma && p.stream) {
    // streaming form: dL/dlogits is formed inside the dx / dwg kernel, per chunk
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const uint16_t* wb = static_cast<const uint16_t*>(wg);
    uint16_t* dxb = static_cast<uint16_t*>(dx_out);
#define MOE_DXDWS(NTEv)                                                                                          \
  launch_dxdw_stream<NTEv>(s, xb, wb, logits, idx, grad_w, gw_dtype, cnt, grad_aux, grad_z, aux_coef, z_coef,    \
                           (int)N, (int)H, (int)E, (int)K, p.tc_len, p.nchunk, dxb, wsdw, nullptr, 0, addb)
    if (p.NTE == 1) MOE_DXDWS(1);
    else MOE_DXDWS(2);
#undef MOE_DXDWS
    if (int rc = check_launch("k_router_dxdw_bf16")) return rc;
    if (dx_add != nullptr && addb == nullptr) launch_add_rows(s, dx_out, dx_add, N * H, x_dtype);
    launch_reduce(s, wsdw, nchunk, H * E, dwg_out, wg_dtype);
    return check_launch("moe_router_bwd");
  }
  if (mfma && p.wide && aligned16(wg)) {
    // wide form: dL/dlogits in bf16 only (16 lanes per token), then the streaming dx / dwg kernel
    const int ekp = p.EK * 32;
#define MOE_GLOGW(EPL)                                                                                         \
  MOE_LAUNCH("k_router_glogits", (k_router_glogits<16, EPL>),                                                  \
             dim3((unsigned)std::min<int64_t>(4096, (N * 16 + 255) / 256)), dim3(256), 0, s, logits, idx,      \
             grad_w, gw_dtype, cnt, grad_aux, grad_z, aux_coef, z_coef, (int)N, (int)E, (int)K, 1,            \
             static_cast<float*>(nullptr), gb, ekp)
    if (E <= 64) MOE_GLOGW(4);
    else MOE_GLOGW(8);
#undef MOE_GLOGW
    if (int rc = check_launch("k_router_glogits")) return rc;
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const uint16_t* wb = static_cast<const uint16_t*>(wg);
    uint16_t* dxb = static_cast<uint16_t*>(dx_out);
    const int nht = (int)(H / 256);
    const dim3 grid((unsigned)(p.nchunk * nht));
    if (p.EK == 2)
      MOE_LAUNCH("k_router_dxdw_bf16", (k_router_dxdw_wide<2, 4>), grid, dim3(256), 0, s, xb, wb, gb, (int)N, (int)H,
                 (int)E, p.tc_len, nht, dxb, addb, wsdw);
    else
      MOE_LAUNCH("k_router_dxdw_bf16", (k_router_dxdw_wide<4, 8>), grid, dim3(256), 0, s, xb, wb, gb, (int)N, (int)H,
                 (int)E, p.tc_len, nht, dxb, addb, wsdw);
    if (int rc = check_launch("k_router_dxdw_bf16")) return rc;
    if (dx_add != nullptr && addb == nullptr) launch_add_rows(s, dx_out, dx_add, N * H, x_dtype);
    launch_reduce(s, wsdw, nchunk, H * E, dwg_out, wg_dtype);
    return check_launch("moe_router_bwd");
  }
  {
    const int ekp = p.EK * 32;
    const int rb = (int)(x_dtype == MOE_BF16);
#define MOE_GLOG(LPT, EPL)                                                                                     \
  MOE_LAUNCH("k_router_glogits", (k_router_glogits<LPT, EPL>),                                                 \
             dim3((unsigned)std::min<int64_t>(4096, (N * LPT + 255) / 256)), dim3(256), 0, s, logits, idx,     \
             grad_w, gw_dtype, cnt, grad_aux, grad_z, aux_coef, z_coef, (int)N, (int)E, (int)K, rb, G, gb, ekp)
    if (E <= 8) MOE_GLOG(8, 1);
    else if (E <= 16) MOE_GLOG(16, 1);
    else if (E <= 32) MOE_GLOG(32, 1);
    else if (E <= 64) MOE_GLOG(64, 1);
    else if (E <= 128) MOE_GLOG(64, 2);
    else MOE_GLOG(64, 4);
#undef MOE_GLOG
  }
  if (int rc = check_launch("k_router_glogits")) return rc;
  if (mfma) {
    const dim3 grid(p.nchunk, cdiv(H, 256));
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    const uint16_t* wb = static_cast<const uint16_t*>(wg);
    uint16_t* dxb = static_cast<uint16_t*>(dx_out);
#define MOE_DXDW(EKv, NTEv) \
  launch_dxdw<EKv, NTEv>(grid, s, xb, wb, gb, (int)N, (int)H, (int)E, p.tc_len, dxb, wsdw)
    if (p.EK == 1 && p.NTE == 1) MOE_DXDW(1, 1);
    else if (p.EK == 1 && p.NTE == 2) MOE_DXDW(1, 2);
    else if (p.EK == 2 && p.NTE == 4) MOE_DXDW(2, 4);
    else if (p.EK == 4 && p.NTE == 8) MOE_DXDW(4, 8);
    else return fail_arg("moe_router_bwd: internal tile error");
#undef MOE_DXDW
    if (int rc = check_launch("k_router_dxdw_bf16")) return rc;
  } else if (p.f32 && aligned16(x) && aligned16(dx_out)) {
    const dim3 grid((unsigned)cdiv(H, 256), (unsigned)p.nchunk);
    const float* xf = static_cast<const float*>(x);
    const float* wf = static_cast<const float*>(wg);
    float* dxf = static_cast<float*>(dx_out);
    if (E <= 8)
      MOE_LAUNCH("k_router_dxdw_f32", k_router_dxdw_f32<8>, grid, dim3(256), 0, s, xf, wf, G, (int)N, (int)H, (int)E,
                 p.tc_len, dxf, wsdw);
    else
      MOE_LAUNCH("k_router_dxdw_f32", k_router_dxdw_f32<16>, grid, dim3(256), 0, s, xf, wf, G, (int)N, (int)H, (int)E,
                 p.tc_len, dxf, wsdw);
    if (int rc = check_launch("k_router_dxdw_f32")) return rc;
  } else {
    const int64_t NH = N * H;
    MOE_LAUNCH("k_router_dx_generic", k_router_dx_generic, dim3((unsigned)std::min<int64_t>(16384, (NH + 255) / 256)), dim3(256), 0,
                       s, G, wg, wg_dtype, (int)N, (int)H, (int)E, dx_out, x_dtype);
    const int64_t he = H * E;
    // the workspace holds p.nchunk partials of p.tc_len tokens each
    const dim3 grid((unsigned)std::min<int64_t>(64, (he + 255) / 256), p.nchunk);
    MOE_LAUNCH("k_router_dw_generic", k_router_dw_generic, grid, dim3(256), 0, s, x, x_dtype, G, (int)N, (int)H, (int)E, p.tc_len,
                       wsdw);
    if (int rc = check_launch("k_router_dw_generic")) return rc;
  }
  // the forms above take no addend: dx += dx_add in a separate pass
  if (dx_add != nullptr) launch_add_rows(s, dx_out, dx_add, N * H, x_dtype);
  const int64_t len = H * E;
  launch_reduce(s,
                     wsdw, nchunk, len, dwg_out, wg_dtype);
  return check_launch("moe_router_bwd");
}

extern "C" int moe_router_bwd(const void* x, int x_dtype, const void* wg, int wg_dtype, const float* logits,
                              const int64_t* idx, const void* grad_w, int gw_dtype, const int64_t* cnt,
                              const float* grad_aux, const float* grad_z, float aux_coef, float z_coef, int64_t N,
                              int64_t H, int64_t E, int64_t K, void* dx_out, void* dwg_out, void* workspace,
                              size_t ws_bytes, void* stream) {
  return moe_router_bwd_acc(x, x_dtype, wg, wg_dtype, logits, idx, grad_w, gw_dtype, cnt, grad_aux, grad_z, aux_coef,
                            z_coef, N, H, E, K, nullptr, dx_out, dwg_out, workspace, ws_bytes, stream);
}
