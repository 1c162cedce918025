// Dispatch planner, permute and combine for gfx950.
//
// Planner: every index structure of the MoE layer is a stable grouping of a
// sequence of items by an integer key -- the rank of item i among earlier
// items with the same key.  Three passes, all deterministic:
//   count  per block of IB items, an LDS histogram (integer atomics, order
//          independent) -> counts[block][key]
//   scan   per key, exclusive prefix over blocks; then exclusive prefix over
//          keys -> key offsets
//   rank   one wave per block walks its items in order, 64 at a time; lanes
//          with equal keys are found with log2(nkeys) ballots (bit-split
//          match), rank-in-chunk = popcount of the lower matching lanes, and a
//          per-key running count in LDS carries the order across chunks.
// Modes (the key of item i):
//   CAPACITY  items = slots t*K+k, key = k*E + idx[t,k]   -> drop = rank >= capacity
//   REFSORT   items = tokens t,    key = idx[t,0]         -> stable sort of column 0
//   ROUTED    items = kept slots,  key = idx[t,k]         -> expert-grouped rows
//
// Permute / combine move whole rows with 16-byte accesses; the combine and
// every backward reduce over the K slots of a token in registers (fp32) with
// a single write, so no float atomics are involved anywhere.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace moe {

enum PlanMode { kCapacity = 0, kRefSort = 1, kRouted = 2 };
constexpr int kPlanIB = 2048;  // items per planner block

// Expert ids are clamped into [0, E) so a malformed index can never address
// outside the planner's tables (the router only produces ids in range).
__device__ __forceinline__ int clamp_e(int64_t v, int E) { return (int)min(max(v, (int64_t)0), (int64_t)(E - 1)); }

__device__ __forceinline__ int plan_key(int mode, const int64_t* __restrict__ idx, int64_t i, int K, int E) {
  if (mode == kCapacity) return (int)(i % K) * E + clamp_e(idx[i], E);
  if (mode == kRefSort) return clamp_e(idx[i * K], E);
  return clamp_e(idx[i], E);
}

__device__ __forceinline__ bool plan_valid(int mode, const uint8_t* __restrict__ drop, int64_t i) {
  return !(mode == kRouted && drop != nullptr && drop[i]);
}

__global__ __launch_bounds__(256) void k_plan_count(int mode, const int64_t* __restrict__ idx,
                                                    const uint8_t* __restrict__ drop, int64_t M, int K, int E,
                                                    int nkeys, int* __restrict__ counts, int* __restrict__ ndrop) {
  extern __shared__ int hist[];
  for (int q = threadIdx.x; q < nkeys; q += blockDim.x) hist[q] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0 && ndrop != nullptr && mode == kCapacity) ndrop[0] = 0;
  __syncthreads();
  const int64_t beg = (int64_t)blockIdx.x * kPlanIB;
  const int64_t end = min(M, beg + kPlanIB);
  for (int64_t i = beg + threadIdx.x; i < end; i += blockDim.x)
    if (plan_valid(mode, drop, i)) atomicAdd(&hist[plan_key(mode, idx, i, K, E)], 1);
  __syncthreads();
  for (int q = threadIdx.x; q < nkeys; q += blockDim.x) counts[(int64_t)blockIdx.x * nkeys + q] = hist[q];
}

// base[b][key] = sum_{b' < b} counts[b'][key]; totals[key] = sum_b counts[b][key].
// Block = 16 keys x 16 block-segments.
__global__ __launch_bounds__(256) void k_plan_scan_blocks(const int* __restrict__ counts, int nblk, int nkeys,
                                                          int* __restrict__ base, int* __restrict__ totals) {
  __shared__ int ss[16][16];
  const int kl = threadIdx.x & 15;
  const int seg = threadIdx.x >> 4;
  const int key = blockIdx.x * 16 + kl;
  const int bps = (nblk + 15) / 16;
  const int b0 = min(nblk, seg * bps);
  const int b1 = min(nblk, b0 + bps);
  int sum = 0;
  if (key < nkeys)
    for (int b = b0; b < b1; ++b) sum += counts[(int64_t)b * nkeys + key];
  ss[seg][kl] = sum;
  __syncthreads();
  if (key < nkeys) {
    int run = 0;
    for (int s = 0; s < seg; ++s) run += ss[s][kl];
    for (int b = b0; b < b1; ++b) {
      base[(int64_t)b * nkeys + key] = run;
      run += counts[(int64_t)b * nkeys + key];
    }
    if (seg == 15) totals[key] = run;
  }
}

// key_off[0..nkeys] = exclusive prefix of totals (one block of 1024 threads).
__global__ __launch_bounds__(1024) void k_plan_scan_keys(const int* __restrict__ totals, int nkeys,
                                                         int* __restrict__ key_off) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int per = (nkeys + 1023) / 1024;
  const int k0 = min(nkeys, tid * per);
  const int k1 = min(nkeys, k0 + per);
  int s = 0;
  for (int k = k0; k < k1; ++k) s += totals[k];
  part[tid] = s;
  __syncthreads();
  // Hillis-Steele inclusive scan over 1024 partials
  for (int o = 1; o < 1024; o <<= 1) {
    const int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = tid ? part[tid - 1] : 0;
  for (int k = k0; k < k1; ++k) {
    key_off[k] = run;
    run += totals[k];
  }
  if (tid == 1023) key_off[nkeys] = part[1023];
}

__global__ __launch_bounds__(64) void k_plan_rank(int mode, const int64_t* __restrict__ idx,
                                                  uint8_t* __restrict__ drop, int64_t M, int K, int E, int nkeys,
                                                  int nbits, const int* __restrict__ base,
                                                  const int* __restrict__ key_off, int64_t capacity,
                                                  int* __restrict__ row_slot, int* __restrict__ slot_row,
                                                  int* __restrict__ ndrop) {
  extern __shared__ int run[];
  const int lane = threadIdx.x;
  for (int q = lane; q < nkeys; q += 64) run[q] = 0;
  __syncthreads();
  const uint64_t lt = (lane == 0) ? 0ull : ((~0ull) >> (64 - lane));
  const int64_t beg = (int64_t)blockIdx.x * kPlanIB;
  const int64_t end = min(M, beg + kPlanIB);
  int dropped = 0;
  for (int64_t c0 = beg; c0 < end; c0 += 64) {
    const int64_t i = c0 + lane;
    const bool active = i < end;
    const bool valid = active && plan_valid(mode, drop, i);
    const int key = valid ? plan_key(mode, idx, i, K, E) : 0;
    uint64_t m = __ballot(valid);
    for (int bit = 0; bit < nbits; ++bit) {
      const bool b = (key >> bit) & 1;
      const uint64_t bm = __ballot(valid && b);
      m &= b ? bm : ~bm;
    }
    if (!valid) m = 0;
    const int rank = __popcll(m & lt);
    const int cnt = __popcll(m);
    const int r = valid ? run[key] : 0;
    __syncthreads();
    if (valid && (m & lt) == 0) run[key] = r + cnt;
    __syncthreads();
    if (!active) continue;
    if (!valid) {  // ROUTED with a dropped slot
      slot_row[i] = -1;
      continue;
    }
    const int pin = base[(int64_t)blockIdx.x * nkeys + key] + r + rank;  // rank among all items of this key
    if (mode == kCapacity) {
      const bool d = (int64_t)pin >= capacity;
      drop[i] = d ? 1 : 0;
      dropped += d ? 1 : 0;
    } else if (mode == kRefSort) {
      const int j = key_off[key] + pin;  // position of token i in the stable sort of column 0
      for (int k = 0; k < K; ++k) {
        row_slot[(int64_t)j * K + k] = (int)(i * K + k);
        slot_row[i * K + k] = j * K + k;
      }
    } else {
      const int row = key_off[key] + pin;
      row_slot[row] = (int)i;
      slot_row[i] = row;
    }
  }
  if (mode == kCapacity) {
    dropped = wave_sum(dropped);
    if (lane == 0 && dropped) atomicAdd(ndrop, dropped);
  }
}

__global__ void k_fill_i32(int* __restrict__ p, int n, int v) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// Reference layout: E equal chunks of chunk = max(1, R / E) rows (rows past E*chunk are never computed).
__global__ void k_plan_ref_offsets(int64_t R, int E, int* __restrict__ offsets) {
  const int64_t chunk = max((int64_t)1, R / E);
  for (int e = threadIdx.x; e <= E; e += blockDim.x) offsets[e] = (int)min((int64_t)e * chunk, R);
}

// Routed layout: rows of dropped slots do not exist; pad row_slot with -1 past the kept rows.
__global__ void k_plan_pad_rows(const int* __restrict__ offsets, int E, int64_t R, int* __restrict__ row_slot) {
  const int64_t kept = offsets[E];
  for (int64_t r = kept + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; r < R; r += (int64_t)gridDim.x * blockDim.x)
    row_slot[r] = -1;
}

// ---------------------------------------------------------------------------
// Permute: xp[r, :] = x[row_slot[r] / K, :] for r < offsets[E].  Byte copy in
// 16-byte units (row_bytes % 16 == 0), one wave per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_permute(const uint8_t* __restrict__ x, const int* __restrict__ row_slot,
                                                 const int* __restrict__ offsets, int E, int K, int64_t row_bytes,
                                                 int64_t R, uint8_t* __restrict__ xp) {
  const int lane = threadIdx.x & 63;
  const int64_t rows = min(R, (int64_t)offsets[E]);
  const int64_t nv = row_bytes / 16;
  for (int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows; r += (int64_t)gridDim.x * 4) {
    const int64_t t = row_slot[r] / K;
    const u32x4* src = reinterpret_cast<const u32x4*>(x + t * row_bytes);
    u32x4* dst = reinterpret_cast<u32x4*>(xp + r * row_bytes);
    for (int64_t v = lane; v < nv; v += 64) __builtin_nontemporal_store(src[v], dst + v);
  }
}

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) {
  return p[i];
}
template <>
__device__ __forceinline__ float ld<uint16_t>(const uint16_t* p, int64_t i) {
  return bf2f(p[i]);
}
template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) {
  p[i] = v;
}
template <>
__device__ __forceinline__ void st<uint16_t>(uint16_t* p, int64_t i, float v) {
  p[i] = f2bf(v);
}

// Streaming store of an 8-element row chunk (rows written once).
template <typename T>
__device__ __forceinline__ void store8_nt(T* p, const float (&f)[8]);
template <>
__device__ __forceinline__ void store8_nt<uint16_t>(uint16_t* p, const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = pack2bf(f[2 * j], f[2 * j + 1]);
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}
template <>
__device__ __forceinline__ void store8_nt<float>(float* p, const float (&f)[8]) {
  __builtin_nontemporal_store(f32x4{f[0], f[1], f[2], f[3]}, reinterpret_cast<f32x4*>(p));
  __builtin_nontemporal_store(f32x4{f[4], f[5], f[6], f[7]}, reinterpret_cast<f32x4*>(p + 4));
}

// 16-byte loads through a buffer descriptor that covers one row: a descriptor with no records (a slot
// without a row) or an offset past the row's end reads zeros without touching memory.  A batch of slot
// loads therefore needs no branch between them, and so no wait for one load before the next issues.
typedef buf_rsrc_t row_rsrc_t;
__device__ __forceinline__ row_rsrc_t row_rsrc(const void* row, int nbytes) { return buf_rsrc(row, nbytes); }
constexpr int kStreamPolicy = 2;  // nt: the rows are read once
template <typename T>
__device__ __forceinline__ void load8_row(row_rsrc_t r, int h0, float (&f)[8]);
template <>
__device__ __forceinline__ void load8_row<uint16_t>(row_rsrc_t r, int h0, float (&f)[8]) {
  const u32x4 v = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, h0 * 2, 0, kStreamPolicy));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[2 * j] = __uint_as_float(v[j] << 16);
    f[2 * j + 1] = __uint_as_float(v[j] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void load8_row<float>(row_rsrc_t r, int h0, float (&f)[8]) {
  const u32x4 a = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, h0 * 4, 0, kStreamPolicy));
  const u32x4 b = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, h0 * 4 + 16, 0, kStreamPolicy));
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = __uint_as_float(a[j]);
    f[4 + j] = __uint_as_float(b[j]);
  }
}

// Slot metadata of one token, one slot per lane: lane l describes slot s0 + l (l < n) -- the
// expert-output row it maps to (-1 when the slot has no computed row: dropped from the plan or
// past offsets[E]), whether the capacity rule dropped it, and its combine weight.  The combine
// loops read a slot's fields from its lane with readlane (wave-uniform values), so every row
// load of a token is addressed without waiting for another load.
struct SlotMeta {
  int row;
  int dropped;
  float w;
};
template <typename TW>
__device__ __forceinline__ float ld_slot_w(row_rsrc_t r, int lane);
template <>
__device__ __forceinline__ float ld_slot_w<float>(row_rsrc_t r, int lane) {
  return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, 0, 0));
}
template <>
__device__ __forceinline__ float ld_slot_w<uint16_t>(row_rsrc_t r, int lane) {
  return __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, lane * 2, 0, 0) << 16);
}
// The three fields are independent buffer loads (absent arrays: descriptors without records), so
// they share one memory round trip.
template <typename TW>
__device__ __forceinline__ SlotMeta slot_meta(const TW* __restrict__ w, const uint8_t* __restrict__ drop,
                                              const int* __restrict__ slot_row, int live_rows, int64_t s0, int n,
                                              int lane) {
  const int r = __builtin_amdgcn_raw_buffer_load_b32(row_rsrc(slot_row + s0, n * 4), lane * 4, 0, 0);
  const int d = __builtin_amdgcn_raw_buffer_load_b8(row_rsrc(drop ? drop + s0 : nullptr, drop ? n : 0), lane, 0, 0);
  const float wt = ld_slot_w<TW>(row_rsrc(w ? w + s0 : nullptr, w ? n * (int)sizeof(TW) : 0), lane);
  SlotMeta m;
  m.row = (lane < n && r >= 0 && r < live_rows) ? r : -1;
  m.dropped = d != 0;
  m.w = wt;
  return m;
}
__device__ __forceinline__ int lane_i(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float lane_f(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// The wave's index in its block as a wave-uniform (scalar) value: the token a wave works on then is
// too, and so are the buffer descriptors built from it.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Slot batching: KG slots (2, 4 or 8: the smallest that covers min(K, 8)) are taken together and
// U = 8 / KG of the lane's 8-element row chunks (512 columns apart) per round, so each round issues
// about 8 independent row loads whatever K is.
template <int KG>
struct SlotBatch {
  static constexpr int U = 8 / KG;
  static constexpr int SPAN = 512 * U;  // columns one round covers
};

// ---------------------------------------------------------------------------
// Combine: out[t, :] = sum_k w[t,k] y[slot_row[t*K+k], :] over the slots that have a computed,
// undropped row (the others contribute nothing).  One wave per token; every row load of a round is
// issued before any is summed.  fp32 sums in slot order, one rounding at the store.
// ---------------------------------------------------------------------------
template <typename T, typename TW, int KG>
__global__ __launch_bounds__(256) void k_combine(const T* __restrict__ y, const TW* __restrict__ w,
                                                 const uint8_t* __restrict__ drop, const int* __restrict__ slot_row,
                                                 const int* __restrict__ offsets, int E, int N, int K, int H,
                                                 T* __restrict__ out) {
  constexpr int U = SlotBatch<KG>::U;
  const int lane = threadIdx.x & 63;
  const int live_rows = offsets[E];
  const int rbytes = H * (int)sizeof(T);
  for (int t = blockIdx.x * 4 + wave_id(); t < N; t += gridDim.x * 4) {
    const int64_t s0 = (int64_t)t * K;
    SlotMeta m = slot_meta(w, drop, slot_row, live_rows, s0, min(K, 64), lane);
    for (int hb = 0; hb < H; hb += SlotBatch<KG>::SPAN) {
      float acc[U][8];
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[u][i] = 0.f;
      for (int kw = 0; kw < K; kw += 64) {
        if (kw > 0) m = slot_meta(w, drop, slot_row, live_rows, s0 + kw, min(K - kw, 64), lane);
        const int kn = min(K - kw, 64);
        for (int kg = 0; kg < kn; kg += KG) {
          int rk[KG];
          float v[KG][U][8];
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            rk[j] = kg + j < kn ? lane_i(m.dropped ? -1 : m.row, kg + j) : -1;
            const row_rsrc_t r = row_rsrc(y + (int64_t)max(rk[j], 0) * H, rk[j] >= 0 ? rbytes : 0);
#pragma unroll
            for (int u = 0; u < U; ++u) load8_row<T>(r, hb + 512 * u + lane * 8, v[j][u]);
          }
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            if (rk[j] < 0) continue;
            const float wk = lane_f(m.w, kg + j);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[u][i] = fmaf(wk, v[j][u][i], acc[u][i]);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int h0 = hb + 512 * u + lane * 8;
        if (h0 < H) store8_nt<T>(out + (int64_t)t * H + h0, acc[u]);
      }
    }
  }
}

// Combine backward: dy[row, :] = w'[t,k] dout[t, :] with w' = 0 for dropped slots, and
// dw[t,k] = <dout[t], y[row]> (0 when dropped); slots without a computed row write no dy and
// dw = 0.  Per batch of KG slots, dout's chunks are loaded once per round together with the
// batch's row chunks; the KG dot products reduce across the wave once the row is done.
template <typename T, typename TW, int KG>
__global__ __launch_bounds__(256) void k_combine_bwd(const T* __restrict__ dout, const T* __restrict__ y,
                                                     const TW* __restrict__ w, const uint8_t* __restrict__ drop,
                                                     const int* __restrict__ slot_row,
                                                     const int* __restrict__ offsets, int E, int N, int K, int H,
                                                     T* __restrict__ dy, TW* __restrict__ dw) {
  constexpr int U = SlotBatch<KG>::U;
  const int lane = threadIdx.x & 63;
  const int live_rows = offsets[E];
  const int rbytes = H * (int)sizeof(T);
  for (int t = blockIdx.x * 4 + wave_id(); t < N; t += gridDim.x * 4) {
    const row_rsrc_t drow = row_rsrc(dout + (int64_t)t * H, rbytes);
    for (int kw = 0; kw < K; kw += 64) {
      const int kn = min(K - kw, 64);
      const SlotMeta m = slot_meta(w, drop, slot_row, live_rows, (int64_t)t * K + kw, kn, lane);
      float mine = 0.f;  // lane l ends with dw of slot kw + l
      for (int kg = 0; kg < kn; kg += KG) {
        int rk[KG];
        float wk[KG], dot[KG];
#pragma unroll
        for (int j = 0; j < KG; ++j) {
          rk[j] = kg + j < kn ? lane_i(m.row, kg + j) : -1;
          wk[j] = lane_i(m.dropped, kg + j) ? 0.f : lane_f(m.w, kg + j);
          dot[j] = 0.f;
        }
        for (int hb = 0; hb < H; hb += SlotBatch<KG>::SPAN) {
          float g[U][8], v[KG][U][8];
#pragma unroll
          for (int u = 0; u < U; ++u) load8_row<T>(drow, hb + 512 * u + lane * 8, g[u]);
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            const row_rsrc_t r = row_rsrc(y + (int64_t)max(rk[j], 0) * H, rk[j] >= 0 ? rbytes : 0);
#pragma unroll
            for (int u = 0; u < U; ++u) load8_row<T>(r, hb + 512 * u + lane * 8, v[j][u]);
          }
          // dy needs only dout: its stores go out before the dot products wait for the rows
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            if (rk[j] < 0) continue;
#pragma unroll
            for (int u = 0; u < U; ++u) {
              const int h0 = hb + 512 * u + lane * 8;
              float o[8];
#pragma unroll
              for (int i = 0; i < 8; ++i) o[i] = wk[j] * g[u][i];
              if (h0 < H) store8_nt<T>(dy + (int64_t)rk[j] * H + h0, o);
            }
          }
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            if (rk[j] < 0) continue;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
              for (int i = 0; i < 8; ++i) dot[j] = fmaf(g[u][i], v[j][u][i], dot[j]);
          }
        }
#pragma unroll
        for (int j = 0; j < KG; ++j) {
          if (rk[j] < 0) continue;
          const float d = wave_sum(dot[j]);
          if (lane == kg + j) mine = d;
        }
      }
      if (lane < kn && dw) st<TW>(dw, (int64_t)t * K + kw + lane, (m.row >= 0 && !m.dropped) ? mine : 0.f);
    }
  }
}

// Permute backward: dx[t, :] = addend[t, :] + sum_k dxp[slot_row[t*K+k], :] over the slots with a
// computed row (dropped slots have none).  Same slot batching as the combine.
template <typename T, int KG>
__global__ __launch_bounds__(256) void k_unpermute_sum(const T* __restrict__ dxp, const T* __restrict__ addend,
                                                       const int* __restrict__ slot_row,
                                                       const int* __restrict__ offsets, int E, int N, int K, int H,
                                                       T* __restrict__ dx) {
  constexpr int U = SlotBatch<KG>::U;
  const int lane = threadIdx.x & 63;
  const int live_rows = offsets[E];
  const int rbytes = H * (int)sizeof(T);
  for (int t = blockIdx.x * 4 + wave_id(); t < N; t += gridDim.x * 4) {
    const int64_t s0 = (int64_t)t * K;
    SlotMeta m = slot_meta<float>(nullptr, nullptr, slot_row, live_rows, s0, min(K, 64), lane);
    const row_rsrc_t arow = row_rsrc(addend ? addend + (int64_t)t * H : dxp, addend ? rbytes : 0);
    for (int hb = 0; hb < H; hb += SlotBatch<KG>::SPAN) {
      float acc[U][8];
#pragma unroll
      for (int u = 0; u < U; ++u) load8_row<T>(arow, hb + 512 * u + lane * 8, acc[u]);  // zeros without an addend
      for (int kw = 0; kw < K; kw += 64) {
        if (kw > 0) m = slot_meta<float>(nullptr, nullptr, slot_row, live_rows, s0 + kw, min(K - kw, 64), lane);
        const int kn = min(K - kw, 64);
        for (int kg = 0; kg < kn; kg += KG) {
          int rk[KG];
          float v[KG][U][8];
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            rk[j] = kg + j < kn ? lane_i(m.row, kg + j) : -1;
            const row_rsrc_t r = row_rsrc(dxp + (int64_t)max(rk[j], 0) * H, rk[j] >= 0 ? rbytes : 0);
#pragma unroll
            for (int u = 0; u < U; ++u) load8_row<T>(r, hb + 512 * u + lane * 8, v[j][u]);
          }
#pragma unroll
          for (int j = 0; j < KG; ++j) {
            if (rk[j] < 0) continue;
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
              for (int i = 0; i < 8; ++i) acc[u][i] += v[j][u][i];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int h0 = hb + 512 * u + lane * 8;
        if (h0 < H) store8_nt<T>(dx + (int64_t)t * H + h0, acc[u]);
      }
    }
  }
}

namespace {

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

struct PlanWs {
  int nblk_max, nkeys_max;
  size_t off_counts, off_base, off_totals, off_keyoff, total;
};

PlanWs plan_ws(int64_t N, int64_t K, int64_t E) {
  PlanWs p{};
  const int64_t M = std::max<int64_t>(1, N * K);
  p.nblk_max = (int)((M + kPlanIB - 1) / kPlanIB);
  p.nkeys_max = (int)(K * E);
  size_t off = 0;
  p.off_counts = off;
  off += al256((size_t)p.nblk_max * p.nkeys_max * 4);
  p.off_base = off;
  off += al256((size_t)p.nblk_max * p.nkeys_max * 4);
  p.off_totals = off;
  off += al256((size_t)p.nkeys_max * 4);
  p.off_keyoff = off;
  off += al256((size_t)(p.nkeys_max + 1) * 4);
  p.total = off;
  return p;
}

int nbits_for(int nkeys) {
  int b = 0;
  while ((1 << b) < nkeys) ++b;
  return b;
}

int grouping(hipStream_t s, int mode, const int64_t* idx, uint8_t* drop, int64_t M, int K, int E, int nkeys,
             int64_t capacity, const PlanWs& p, char* ws, int* key_off_out, int* row_slot, int* slot_row,
             int* ndrop) {
  const int nblk = (int)((M + kPlanIB - 1) / kPlanIB);
  int* counts = reinterpret_cast<int*>(ws + p.off_counts);
  int* base = reinterpret_cast<int*>(ws + p.off_base);
  int* totals = reinterpret_cast<int*>(ws + p.off_totals);
  int* key_off = key_off_out ? key_off_out : reinterpret_cast<int*>(ws + p.off_keyoff);
  const size_t lds = (size_t)nkeys * 4;
  MOE_LAUNCH("k_plan_count", k_plan_count, dim3(nblk), dim3(256), lds, s, mode, idx, drop, M, K, E, nkeys, counts,
             ndrop);
  MOE_LAUNCH("k_plan_scan_blocks", k_plan_scan_blocks, dim3((nkeys + 15) / 16), dim3(256), 0, s, counts, nblk, nkeys,
             base, totals);
  MOE_LAUNCH("k_plan_scan_keys", k_plan_scan_keys, dim3(1), dim3(1024), 0, s, totals, nkeys, key_off);
  MOE_LAUNCH("k_plan_rank", k_plan_rank, dim3(nblk), dim3(64), lds, s, mode, idx, drop, M, K, E, nkeys,
             nbits_for(nkeys), base, key_off, capacity, row_slot, slot_row, ndrop);
  return check_launch("moe_plan grouping");
}

bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_plan_workspace(int64_t N, int64_t K, int64_t E) {
  if (N <= 0 || K <= 0 || E <= 0) return 0;
  return plan_ws(N, K, E).total;
}

namespace moe {
namespace {

int plan_check(int64_t N, int64_t K, int64_t E, int layout, const int32_t* offsets, const int32_t* ndrop) {
  if (N < 0 || K < 1 || E < 1 || K > E || E > 1024 || K * E > 8192)
    return fail_arg("moe_plan: bad shape N=%lld K=%lld E=%lld", (long long)N, (long long)K, (long long)E);
  if (N * K > INT32_MAX / 2) return fail_arg("moe_plan: N*K too large");
  if (layout != 0 && layout != 1) return fail_arg("moe_plan: layout must be 0 (reference) or 1 (routed)");
  if (!offsets || !ndrop) return fail_arg("moe_plan: null offsets/ndrop");
  return 0;
}

// The plan proper, with its block tables in `ws` (plan_ws(N, K, E).total bytes; every table is written
// before it is read, so ws needs no initialisation).
int plan_run(const int64_t* idx, int64_t N, int64_t K, int64_t E, int64_t capacity, int layout, uint8_t* drop_out,
             int32_t* row_slot, int32_t* slot_row, int32_t* offsets, int32_t* ndrop, char* ws, hipStream_t s) {
  const int64_t M = N * K;
  const PlanWs p = plan_ws(N, K, E);
  uint8_t* drop = capacity >= 0 ? drop_out : nullptr;
  if (drop) {
    if (int rc = grouping(s, kCapacity, idx, drop, M, (int)K, (int)E, (int)(K * E), capacity, p, ws, nullptr,
                          row_slot, slot_row, ndrop))
      return rc;
  } else {
    MOE_LAUNCH("k_fill_i32", k_fill_i32, dim3(1), dim3(64), 0, s, ndrop, 1, 0);
  }
  if (layout == 0) {
    if (int rc = grouping(s, kRefSort, idx, nullptr, N, (int)K, (int)E, (int)E, -1, p, ws, nullptr, row_slot,
                          slot_row, ndrop))
      return rc;
    MOE_LAUNCH("k_plan_ref_offsets", k_plan_ref_offsets, dim3(1), dim3(256), 0, s, M, (int)E, offsets);
  } else {
    if (int rc = grouping(s, kRouted, idx, drop, M, (int)K, (int)E, (int)E, -1, p, ws, offsets, row_slot, slot_row,
                          ndrop))
      return rc;
    MOE_LAUNCH("k_plan_pad_rows", k_plan_pad_rows, dim3((unsigned)std::min<int64_t>(1024, (M + 255) / 256)),
               dim3(256), 0, s, offsets, (int)E, M, row_slot);
  }
  return check_launch("moe_plan");
}

// An empty plan (N * K == 0): zero offsets and drop count.
int plan_empty(int64_t E, int32_t* offsets, int32_t* ndrop, hipStream_t s) {
  MOE_LAUNCH("k_fill_i32", k_fill_i32, dim3(1), dim3(256), 0, s, offsets, (int)(E + 1), 0);
  MOE_LAUNCH("k_fill_i32", k_fill_i32, dim3(1), dim3(64), 0, s, ndrop, 1, 0);
  return check_launch("moe_plan");
}

}  // namespace
}  // namespace moe

extern "C" int moe_plan(const int64_t* idx, int64_t N, int64_t K, int64_t E, int64_t capacity, int layout,
                        uint8_t* drop_out, int32_t* row_slot, int32_t* slot_row, int32_t* offsets, int32_t* ndrop,
                        void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = plan_check(N, K, E, layout, offsets, ndrop)) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (N * K == 0) return plan_empty(E, offsets, ndrop, s);
  if (!idx || !row_slot || !slot_row) return fail_arg("moe_plan: null pointer argument");
  if (capacity >= 0 && !drop_out) return fail_arg("moe_plan: capacity dropping needs drop_out");
  const PlanWs p = plan_ws(N, K, E);
  if (ws_bytes < p.total || !workspace)
    return set_error("moe_plan: workspace %zu < %zu bytes", ws_bytes, p.total), MOE_EWORKSPACE;
  return plan_run(idx, N, K, E, capacity, layout, drop_out, row_slot, slot_row, offsets, ndrop,
                  static_cast<char*>(workspace), s);
}

// ---------------------------------------------------------------------------
// Allocation-free planner: the block tables live in `scratch`, a fixed device array of this library
// (each GPU holds its own copy, from the library's load until the process ends).  In host code `scratch`
// names a host-side stand-in, not device memory: its device address is looked up once per device with
// hipGetSymbolAddress and only that address is handed to the kernels.
// ---------------------------------------------------------------------------
static __device__ __align__(256) char scratch[MOE_PLAN_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// Device address of the current device's `scratch` (looked up on the first call on that device).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error("moe_plan_noalloc: hipGetDevice: %s", hipGetErrorString(e)), (int)e;
  if (dev < 0 || dev >= kMaxDevices) return fail_arg("moe_plan_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error("moe_plan_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e)),
             e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return 0;
}
}  // namespace

extern "C" int moe_plan_noalloc(const int64_t* idx, int64_t N, int64_t K, int64_t E, int64_t capacity, int layout,
                                uint8_t* drop_out, int32_t* row_slot, int32_t* slot_row, int32_t* offsets,
                                int32_t* ndrop, void* stream) {
  if (int rc = plan_check(N, K, E, layout, offsets, ndrop)) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (N * K == 0) return plan_empty(E, offsets, ndrop, s);
  if (!idx || !row_slot || !slot_row) return fail_arg("moe_plan_noalloc: null pointer argument");
  if (capacity >= 0 && !drop_out) return fail_arg("moe_plan_noalloc: capacity dropping needs drop_out");
  const PlanWs p = plan_ws(N, K, E);
  if (p.total > (size_t)MOE_PLAN_SCRATCH_BYTES)
    return fail_arg("moe_plan_noalloc: N=%lld K=%lld E=%lld needs %zu bytes of block tables, more than the %d-byte "
                    "scratch array (use moe_plan with a workspace)", (long long)N, (long long)K, (long long)E,
                    p.total, MOE_PLAN_SCRATCH_BYTES);
  void* ptr = nullptr;
  if (int rc = scratch_address(&ptr)) return rc;
  return plan_run(idx, N, K, E, capacity, layout, drop_out, row_slot, slot_row, offsets, ndrop,
                  static_cast<char*>(ptr), s);
}

extern "C" int moe_permute(const void* x, int64_t row_bytes, const int32_t* row_slot, const int32_t* offsets,
                           int64_t E, int64_t K, int64_t R, void* xp, void* stream) {
  if (row_bytes <= 0 || row_bytes % 16 || E < 1 || K < 1 || R < 0)
    return fail_arg("moe_permute: bad arguments (row_bytes must be a positive multiple of 16)");
  if (R == 0) return 0;
  if (!x || !row_slot || !offsets || !xp || !al16(x) || !al16(xp))
    return fail_arg("moe_permute: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned nb = (unsigned)std::min<int64_t>(8192, (R + 3) / 4);
  MOE_LAUNCH("k_permute", k_permute, dim3(nb), dim3(256), 0, s, static_cast<const uint8_t*>(x), row_slot, offsets,
             (int)E, (int)K, row_bytes, R, static_cast<uint8_t*>(xp));
  return check_launch("moe_permute");
}

// Slot batch of the combine kernels: the smallest of 2, 4, 8 that covers min(K, 8).
#define MOE_KG(k, KERNEL_CALL)                                   \
  do {                                                           \
    if ((k) <= 2) { constexpr int KG = 2; KERNEL_CALL; }         \
    else if ((k) <= 4) { constexpr int KG = 4; KERNEL_CALL; }    \
    else { constexpr int KG = 8; KERNEL_CALL; }                  \
  } while (0)

#define MOE_DT2(dt, dtw, KERNEL_CALL)                                              \
  do {                                                                            \
    if (dt == MOE_BF16 && dtw == MOE_BF16) { using T = uint16_t; using TW = uint16_t; KERNEL_CALL; } \
    else if (dt == MOE_BF16 && dtw == MOE_F32) { using T = uint16_t; using TW = float; KERNEL_CALL; } \
    else if (dt == MOE_F32 && dtw == MOE_F32) { using T = float; using TW = float; KERNEL_CALL; }     \
    else { using T = float; using TW = uint16_t; KERNEL_CALL; }                   \
  } while (0)

extern "C" int moe_combine(const void* y, int dtype, const void* w, int w_dtype, const uint8_t* drop,
                           const int32_t* slot_row, const int32_t* offsets, int64_t N, int64_t K, int64_t H,
                           int64_t E, void* out, void* stream) {
  if (N < 0 || K < 1 || H < 8 || H % 8 || E < 1) return fail_arg("moe_combine: bad shape (H must be a multiple of 8)");
  if ((dtype != MOE_F32 && dtype != MOE_BF16) || (w_dtype != MOE_F32 && w_dtype != MOE_BF16))
    return fail_arg("moe_combine: unsupported dtype");
  if (N == 0) return 0;
  if (!y || !w || !slot_row || !offsets || !out || !al16(y) || !al16(out))
    return fail_arg("moe_combine: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned nb = (unsigned)std::min<int64_t>(8192, (N + 3) / 4);
  MOE_DT2(dtype, w_dtype, MOE_KG(K,
          MOE_LAUNCH("k_combine", (k_combine<T, TW, KG>), dim3(nb), dim3(256), 0, s, static_cast<const T*>(y),
                     static_cast<const TW*>(w), drop, slot_row, offsets, (int)E, (int)N, (int)K, (int)H,
                     static_cast<T*>(out))));
  return check_launch("moe_combine");
}

extern "C" int moe_combine_bwd(const void* dout, const void* y, int dtype, const void* w, int w_dtype,
                               const uint8_t* drop, const int32_t* slot_row, const int32_t* offsets, int64_t N,
                               int64_t K, int64_t H, int64_t E, void* dy, void* dw, void* stream) {
  if (N < 0 || K < 1 || H < 8 || H % 8 || E < 1)
    return fail_arg("moe_combine_bwd: bad shape (H must be a multiple of 8)");
  if ((dtype != MOE_F32 && dtype != MOE_BF16) || (w_dtype != MOE_F32 && w_dtype != MOE_BF16))
    return fail_arg("moe_combine_bwd: unsupported dtype");
  if (N == 0) return 0;
  if (!dout || !y || !w || !slot_row || !offsets || !dy || !al16(dout) || !al16(y) || !al16(dy))
    return fail_arg("moe_combine_bwd: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned nb = (unsigned)std::min<int64_t>(8192, (N + 3) / 4);
  MOE_DT2(dtype, w_dtype, MOE_KG(K,
          MOE_LAUNCH("k_combine_bwd", (k_combine_bwd<T, TW, KG>), dim3(nb), dim3(256), 0, s, static_cast<const T*>(dout),
                     static_cast<const T*>(y), static_cast<const TW*>(w), drop, slot_row, offsets, (int)E, (int)N,
                     (int)K, (int)H, static_cast<T*>(dy), static_cast<TW*>(dw))));
  return check_launch("moe_combine_bwd");
}

extern "C" int moe_unpermute_sum(const void* dxp, const void* addend, int dtype, const int32_t* slot_row,
                                 const int32_t* offsets, int64_t N, int64_t K, int64_t H, int64_t E, void* dx,
                                 void* stream) {
  if (N < 0 || K < 1 || H < 8 || H % 8 || E < 1)
    return fail_arg("moe_unpermute_sum: bad shape (H must be a multiple of 8)");
  if (dtype != MOE_F32 && dtype != MOE_BF16) return fail_arg("moe_unpermute_sum: unsupported dtype");
  if (N == 0) return 0;
  if (!dxp || !slot_row || !offsets || !dx || !al16(dxp) || !al16(dx) || (addend && !al16(addend)))
    return fail_arg("moe_unpermute_sum: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned nb = (unsigned)std::min<int64_t>(8192, (N + 3) / 4);
  if (dtype == MOE_BF16)
    MOE_KG(K, MOE_LAUNCH("k_unpermute_sum", (k_unpermute_sum<uint16_t, KG>), dim3(nb), dim3(256), 0, s,
                         static_cast<const uint16_t*>(dxp), static_cast<const uint16_t*>(addend), slot_row, offsets,
                         (int)E, (int)N, (int)K, (int)H, static_cast<uint16_t*>(dx)));
  else
    MOE_KG(K, MOE_LAUNCH("k_unpermute_sum", (k_unpermute_sum<float, KG>), dim3(nb), dim3(256), 0, s,
                         static_cast<const float*>(dxp), static_cast<const float*>(addend), slot_row, offsets, (int)E,
                         (int)N, (int)K, (int)H, static_cast<float*>(dx)));
  return check_launch("moe_unpermute_sum");
}
