// Dispatch planner, permute and combine for gfx950.
//
// Planner: every index structure of the MoE layer is a stable grouping of a
// sequence of items by an integer key -- the rank of item i among earlier
// items with the same key.  Inside one block the items are split into one
// contiguous part per wave; each wave loads its part's keys into registers
// (one memory round trip), counts them per key (lanes with equal keys are
// found with log2(nkeys) ballots, a bit-split match), the per-wave counts are
// prefixed over waves, and a second walk over the registers gives each item
// its rank: the wave's running count + the popcount of the lower matching
// lanes.  Small plans run in one block; larger ones in three launches per
// grouping, all deterministic:
//   count  per block of IB items, an LDS histogram -> counts[key][block]
//   scan   one wave per key: exclusive prefix over blocks, key totals
//   rank   per block: key offsets (prefix of the totals), in-block ranks
// Modes (the key of item i):
//   CAPACITY  items = slots t*K+k, key = k*E + idx[t,k]   -> drop = rank >= capacity
//   REFSORT   items = tokens t,    key = idx[t,0]         -> stable sort of column 0
//   ROUTED    items = kept slots,  key = idx[t,k]         -> expert-grouped rows
//
// Permute / combine move whole rows with 16-byte accesses; the combine and
// every backward reduce over the K slots of a token in registers (fp32) with
// a single write, so no float atomics are involved anywhere.
#include <algorithm>
#include <atomic>
#include <mutex>

#include "common.h"

namespace moe {

enum PlanMode { kCapacity = 0, kRefSort = 1, kRouted = 2 };
constexpr int kPlanIB = 2048;  // items per planner block
constexpr int kPlanMaxK = 128;  // largest top-k of the fused capacity + routed path

// Expert ids are clamped into [0, E) so a malformed index can never address
// outside the planner's tables (the router only produces ids in range).
__device__ __forceinline__ int clamp_e(int64_t v, int E) { return (int)min(max(v, (int64_t)0), (int64_t)(E - 1)); }

__host__ __device__ __attribute__((always_inline)) inline int nbits_of(int nkeys) {
  int b = 0;
  while ((1 << b) < nkeys) ++b;
  return b;
}

// ---------------------------------------------------------------------------
// Stable grouping inside one 1024-thread block.  The items of a range are split into nwr contiguous parts,
// one per wave (waves past nwr idle: nwr shrinks with the key count so the per-wave key counts fit in LDS).
//   pass 1  each wave walks its part in chunks of 64 and counts its items per key: lanes with equal keys
//           are found with log2(nkeys) ballots (bit-split match); the lowest lane of each key group adds
//           the group's size to cnt[w][key] (an LDS integer add not waited on: the sums do not depend on
//           the order)
//   prefix  per key, exclusive prefix of cnt[.][key] over the waves (tot[key] = the range's total)
//   pass 2  each wave walks its part again: an item's rank among the range's items of its key is
//           cnt[w][key] (running) + its rank among the equal-keyed lanes of its chunk
// Ranks therefore follow the item order exactly, and the result is independent of timing.
// ---------------------------------------------------------------------------
constexpr int kPlanNT = 1024;            // threads of a planner block (16 waves)
constexpr int kPlanSmall = 16384;        // largest item count the single-block planner takes
constexpr int kPlanCntInts = 24576;      // LDS ints of the per-wave key counts (96 KB)

__host__ __device__ __attribute__((always_inline)) constexpr int plan_nwr(int nkeys) {
  int w = 16;
  while (w > 1 && w * nkeys > kPlanCntInts) w >>= 1;
  return w;
}

__device__ __forceinline__ uint64_t key_match(bool valid, int key, int nbits) {
  uint64_t m = __ballot(valid);
  for (int bit = 0; bit < nbits; ++bit) {
    const bool b = (key >> bit) & 1;
    const uint64_t bm = __ballot(valid && b);
    m &= b ? bm : ~bm;
  }
  return valid ? m : 0ull;
}

// Per-mode keys (items: slots t*K+k for CAPACITY and ROUTED, tokens t for REFSORT).  Item i's expert id is read
// at idx[i * stride] (and ROUTED's drop flag at drop[i]); key() turns them into the item's key, -1 for an
// item without one (a dropped slot).
struct PlanKeys {
  const int64_t* idx;
  const uint8_t* drop;  // ROUTED: dropped slots have no key (null: none dropped)
  int K, E;
  __device__ __forceinline__ int64_t stride(int mode) const { return mode == kRefSort ? K : 1; }
  __device__ __forceinline__ int key(int mode, int64_t i, int64_t e, int d) const {
    const int ce = clamp_e(e, E);
    if (mode == kCapacity) return ((int)i % K) * E + ce;  // i < 2^31 (N*K is bounded on the host)
    return (mode == kRouted && d) ? -1 : ce;
  }
};

// A wave's part of a range, its keys loaded into registers first (one round of loads for both passes): chunk c
// of the part covers items lo + 64 c + lane; key[c] = the item's key, -1 for an item without one (ROUTED: a
// dropped slot), -2 past the part.
constexpr int kPlanCh = 16;  // chunks a wave holds (the part of a wave is at most 64 * kPlanCh items)
// a multi-block rank pass splits kPlanIB items over plan_nwr(nkeys) waves; nkeys <= 8192 (K*E)
static_assert(plan_nwr(8192) * 64 * kPlanCh >= kPlanIB, "a rank block's items must fit its waves");
static_assert(8192 <= 8 * kPlanNT, "a rank block's threads hold at most 8 keys each");

struct WaveKeys {
  int key[kPlanCh];
  int64_t lo;
  int nch;
};

// Every load is issued before any key is formed (clamped addresses: lanes past the range re-read its last
// item), so the part's keys cost one memory round trip.
__device__ __forceinline__ void load_keys(WaveKeys& wk, int64_t beg, int64_t end, int nwr, int w, int lane,
                                          const PlanKeys& pk, int mode) {
  const int64_t part = (((end - beg) + (int64_t)nwr * 64 - 1) / ((int64_t)nwr * 64)) * 64;
  wk.lo = beg + (int64_t)w * part;
  const int64_t hi = min(end, wk.lo + part);
  wk.nch = hi > wk.lo ? (int)((hi - wk.lo + 63) / 64) : 0;
  const int64_t st = pk.stride(mode);
  const uint8_t* dp = mode == kRouted ? pk.drop : nullptr;
  int64_t e[kPlanCh];
  int d[kPlanCh];
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) e[c] = pk.idx[min(wk.lo + 64 * c + lane, end - 1) * st];
  if (dp) {
#pragma unroll
    for (int c = 0; c < kPlanCh; ++c) d[c] = dp[min(wk.lo + 64 * c + lane, end - 1)];
  } else {
#pragma unroll
    for (int c = 0; c < kPlanCh; ++c) d[c] = 0;
  }
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) {
    const int64_t i = wk.lo + 64 * c + lane;
    wk.key[c] = (c < wk.nch && i < hi) ? pk.key(mode, i, e[c], d[c]) : -2;
  }
}

// pass 1 (wave w < nwr): cnt[w * nkeys + key] = items of the wave's part with that key (cnt starts zeroed)
__device__ __forceinline__ void group_count(const WaveKeys& wk, int w, int lane, int nkeys, int nbits, int* cnt) {
  const uint64_t lt = lane ? ((~0ull) >> (64 - lane)) : 0ull;
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) {
    if (c < wk.nch) {  // wave-uniform
      const int key = wk.key[c];
      const bool valid = key >= 0;
      const uint64_t m = key_match(valid, key, nbits);
      if (valid && (m & lt) == 0) atomicAdd(&cnt[w * nkeys + key], __popcll(m));  // no return: not waited on
    }
  }
}

// prefix: cnt[w][key] <- sum_{w' < w} cnt[w'][key]; tot[key] <- sum over all waves (tot may be null).  A key's
// nwr <= 16 counts are read before any is written.
__device__ __forceinline__ void group_prefix(int nwr, int nkeys, int* cnt, int* tot) {
  for (int key = threadIdx.x; key < nkeys; key += blockDim.x) {
    int v[16];
#pragma unroll
    for (int w = 0; w < 16; ++w) v[w] = w < nwr ? cnt[w * nkeys + key] : 0;
    int run = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
      if (w < nwr) cnt[w * nkeys + key] = run;
      run += v[w];
    }
    if (tot) tot[key] = run;
  }
}

// pass 2 (wave w < nwr): out(i, key, rank) for each item with a key, skip(i) for each item without one
template <class Out, class Skip>
__device__ __forceinline__ void group_rank(const WaveKeys& wk, int w, int lane, int nkeys, int nbits, int* cnt,
                                           Out out, Skip skip) {
  const uint64_t lt = lane ? ((~0ull) >> (64 - lane)) : 0ull;
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) {
    if (c < wk.nch) {  // wave-uniform
      const int key = wk.key[c];
      const int64_t i = wk.lo + 64 * c + lane;
      const bool valid = key >= 0;
      const uint64_t m = key_match(valid, key, nbits);
      const int run = valid ? cnt[w * nkeys + key] : 0;
      if (valid) out(i, key, run + __popcll(m & lt));
      else if (key == -1) skip(i);
      // the running count moves on only after every lane of the key group has read it (a wave's LDS
      // operations complete in order)
      if (valid && (m & lt) == 0) cnt[w * nkeys + key] = run + __popcll(m);
    }
  }
}

// pass 2 of a grouping whose items then take part in a second grouping of the same parts: wk.key[c] <-
// rekey(i, key, rank) for each item with a key (items without one keep theirs)
template <class Rekey>
__device__ __forceinline__ void group_rank_rekey(WaveKeys& wk, int w, int lane, int nkeys, int nbits, int* cnt,
                                                 Rekey rekey) {
  const uint64_t lt = lane ? ((~0ull) >> (64 - lane)) : 0ull;
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) {
    if (c < wk.nch) {  // wave-uniform
      const int key = wk.key[c];
      const int64_t i = wk.lo + 64 * c + lane;
      const bool valid = key >= 0;
      const uint64_t m = key_match(valid, key, nbits);
      const int run = valid ? cnt[w * nkeys + key] : 0;
      if (valid) wk.key[c] = rekey(i, key, run + __popcll(m & lt));
      if (valid && (m & lt) == 0) cnt[w * nkeys + key] = run + __popcll(m);
    }
  }
}

// exclusive prefix of tot[0..n) into off[0..n] (off[n] = total), ending with a block barrier.  Up to 1024 keys
// wave 0 does it alone (at most 16 keys per lane, one wave scan, no barrier inside); beyond, the whole
// 1024-thread block (part: LDS [1024]).
__device__ __forceinline__ void block_excl_scan(const int* tot, int n, int* off, int* part) {
  const int tid = threadIdx.x;
  if (n <= 64 * 16) {
    if (tid < 64) {
      const int per = (n + 63) / 64;
      const int k0 = min(n, tid * per), k1 = min(n, k0 + per);
      int sum = 0;
      for (int k = k0; k < k1; ++k) sum += tot[k];
      int incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (tid >= o) incl += t;
      }
      int run = incl - sum;
      for (int k = k0; k < k1; ++k) {
        off[k] = run;
        run += tot[k];
      }
      if (tid == 63) off[n] = incl;
    }
    __syncthreads();
    return;
  }
  const int per = (n + kPlanNT - 1) / kPlanNT;
  const int k0 = min(n, tid * per), k1 = min(n, k0 + per);
  int sum = 0;
  for (int k = k0; k < k1; ++k) sum += tot[k];
  part[tid] = sum;
  __syncthreads();
  for (int o = 1; o < kPlanNT; o <<= 1) {
    const int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int run = tid ? part[tid - 1] : 0;
  for (int k = k0; k < k1; ++k) {
    off[k] = run;
    run += tot[k];
  }
  if (tid == kPlanNT - 1) off[n] = part[kPlanNT - 1];
  __syncthreads();
}

__device__ __forceinline__ int block_sum(int v, int* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  int t = 0;
  for (int q = 0; q < (int)(blockDim.x >> 6); ++q) t += red[q];
  __syncthreads();
  return t;
}

// Largest item count of one wave-split range (the part of a wave holds at most kPlanCh chunks of 64).
__host__ __device__ inline int64_t plan_range_max(int nkeys) { return (int64_t)plan_nwr(nkeys) * 64 * kPlanCh; }

// LDS of the single-block planner (ints).  The capacity grouping's per-wave counts [nwr(K*E) * K*E] start at 0;
// the layout grouping's arrays -- cnt [nwr(E) * E], tot [E], off [E + 1], part [1024], red [16] -- and the row
// table staged for coalesced stores [M] follow them in the same space once the capacity pass is done.
__host__ __device__ inline int plan_small_base(int E) { return plan_nwr(E) * E + 2 * E + 1 + kPlanNT + 16; }
__host__ __device__ inline int64_t plan_small_lds_ints(int64_t M, int K, int E, bool drops) {
  const int64_t a = drops ? (int64_t)plan_nwr(K * E) * K * E : 0;
  const int64_t b = plan_small_base(E) + M;
  return a > b ? a : b;
}

// The single-block planner takes N*K <= kPlanSmall items when every grouping's range fits its waves.
__host__ __device__ inline bool plan_small_ok(int64_t M, int K, int E, bool drops) {
  return M <= kPlanSmall && (!drops || M <= plan_range_max(K * E)) && M <= plan_range_max(E) &&
         plan_small_lds_ints(M, K, E, drops) * 4 <= 160 * 1024;
}

// Rank callbacks of the layouts, shared by the single-block and the multi-block planner.  koff: key offsets;
// bbase(key): the key's items in earlier blocks (0 in the single-block planner).
struct RefOut {  // REFSORT: token t at position j of the stable sort of column 0 takes rows j*K .. j*K+K-1
  int K;
  int* row_slot;
  int* slot_row;
  __device__ __forceinline__ void operator()(int64_t t, int64_t j) const {
    for (int k = 0; k < K; ++k) {
      row_slot[j * K + k] = (int)(t * K + k);
      slot_row[t * K + k] = (int)(j * K + k);
    }
  }
};

// The whole plan in one block, for plan_small_ok: capacity drops (optional), then the reference or the routed
// row layout, every table in LDS (plan_small_lds_ints).  The row table's ranks scatter over M rows, so its
// entries are staged in LDS and stored in order at the end (16-byte stores); slot_row is written in item order.
__global__ __launch_bounds__(kPlanNT) void k_plan_small(const int64_t* __restrict__ idx, int N, int K, int E,
                                                        int64_t capacity, int layout, uint8_t* __restrict__ drop,
                                                        int* __restrict__ row_slot, int* __restrict__ slot_row,
                                                        int* __restrict__ offsets, int* __restrict__ ndrop) {
  extern __shared__ int lds[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int M = N * K;  // <= kPlanSmall
  const int nkeys = E, nwr = plan_nwr(E), nbits = nbits_of(E);
  int* cnt = lds;
  int* tot = cnt + nwr * nkeys;
  int* off = tot + nkeys;
  int* part = off + nkeys + 1;
  int* red = part + kPlanNT;
  int* stage = red + 16;
  PlanKeys pk{idx, capacity >= 0 ? drop : nullptr, K, E};
  WaveKeys wk;
  if (capacity >= 0) {
    int* ccnt = lds;
    const int cnk = K * E, cnw = plan_nwr(cnk), cnb = nbits_of(cnk);
    if (w < cnw) load_keys(wk, 0, M, cnw, w, lane, pk, kCapacity);
    for (int q = threadIdx.x; q < cnw * cnk; q += kPlanNT) ccnt[q] = 0;
    __syncthreads();
    if (w < cnw) group_count(wk, w, lane, cnk, cnb, ccnt);
    __syncthreads();
    group_prefix(cnw, cnk, ccnt, nullptr);
    __syncthreads();
    int dropped = 0;
    if (w < cnw)
      group_rank(wk, w, lane, cnk, cnb, ccnt,
                 [&](int64_t i, int, int rank) {
                   const bool d = (int64_t)rank >= capacity;
                   drop[i] = d ? 1 : 0;
                   dropped += d ? 1 : 0;
                 },
                 [](int64_t) {});
    __syncthreads();  // the drops are visible to the whole block (workgroup-scope fence); ccnt is dead
    const int total_dropped = block_sum(dropped, red);
    if (threadIdx.x == 0) ndrop[0] = total_dropped;
  } else if (threadIdx.x == 0) {
    ndrop[0] = 0;
  }
  const int nitems = layout == 0 ? N : M;
  const int lmode = layout == 0 ? kRefSort : kRouted;
  // item i takes position pos of the grouping: the reference layout gives token i (a position of the stable
  // sort of column 0) rows pos*K .. pos*K+K-1; the routed layout gives slot i row pos
  auto place = [&](int64_t i, int pos) {
    if (layout == 0) {
      for (int k = 0; k < K; ++k) {
        stage[pos * K + k] = (int)i * K + k;
        slot_row[i * K + k] = pos * K + k;
      }
    } else {
      stage[pos] = (int)i;
      slot_row[i] = pos;
    }
  };
  auto skip = [&](int64_t i) { slot_row[i] = -1; };  // a dropped slot (routed layout)
  if (w < nwr) load_keys(wk, 0, nitems, nwr, w, lane, pk, lmode);
  for (int q = threadIdx.x; q < nwr * nkeys; q += kPlanNT) cnt[q] = 0;
  __syncthreads();
  if (w < nwr) group_count(wk, w, lane, nkeys, nbits, cnt);
  __syncthreads();
  group_prefix(nwr, nkeys, cnt, tot);
  __syncthreads();
  block_excl_scan(tot, nkeys, off, part);
  if (w < nwr)
    group_rank(wk, w, lane, nkeys, nbits, cnt, [&](int64_t i, int key, int rank) { place(i, off[key] + rank); },
               skip);
  __syncthreads();  // the staged row table and the key offsets are complete
  if (layout == 0) {
    const int64_t chunk = max((int64_t)1, (int64_t)M / E);  // E equal chunks; rows past E*chunk are never computed
    for (int e = threadIdx.x; e <= E; e += kPlanNT) offsets[e] = (int)min((int64_t)e * chunk, (int64_t)M);
  } else {
    for (int e = threadIdx.x; e <= E; e += kPlanNT) offsets[e] = off[e];
  }
  const int kept = layout == 0 ? M : off[E];  // rows past the kept ones (routed layout) have no slot: -1
  if ((reinterpret_cast<uintptr_t>(row_slot) & 15u) == 0) {
    for (int r = 4 * (int)threadIdx.x; r < M; r += 4 * kPlanNT) {
      if (r + 4 <= M) {
        int4 v;
        v.x = r < kept ? stage[r] : -1;
        v.y = r + 1 < kept ? stage[r + 1] : -1;
        v.z = r + 2 < kept ? stage[r + 2] : -1;
        v.w = r + 3 < kept ? stage[r + 3] : -1;
        *reinterpret_cast<int4*>(row_slot + r) = v;
      } else {
        for (int q = r; q < M; ++q) row_slot[q] = q < kept ? stage[q] : -1;
      }
    }
  } else {
    for (int r = threadIdx.x; r < M; r += kPlanNT) row_slot[r] = r < kept ? stage[r] : -1;
  }
}

// Few keys without capacity drops (E <= kPlanByKey, N*K <= kPlanSmall): block k of E places the items whose key
// is k, so the grouping runs on E CUs at once.  Every block loads all the keys (16 waves, coalesced; L2 serves
// all but the first block), counts per wave the items with a smaller key (-> the key's offset) and those with
// key k (-> each wave's base), then ranks its items chunk by chunk with one ballot: rank = offset + wave base +
// earlier chunks + lower lanes.  Item order is (wave, chunk, lane), so the ranks are the stable order.  Block k
// writes only its own rows (a contiguous range of row_slot) and its items' slot_row entries.
constexpr int kPlanByKey = 16;
__global__ __launch_bounds__(kPlanNT) void k_plan_bykey(const int64_t* __restrict__ idx, int N, int K, int E,
                                                        int layout, int* __restrict__ row_slot,
                                                        int* __restrict__ slot_row, int* __restrict__ offsets,
                                                        int* __restrict__ ndrop) {
  __shared__ int s_lt[kPlanNT / 64], s_eq[kPlanNT / 64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int key = blockIdx.x;
  const int M = N * K;
  const int nitems = layout == 0 ? N : M;
  const PlanKeys pk{idx, nullptr, K, E};
  WaveKeys wk;
  load_keys(wk, 0, nitems, kPlanNT / 64, w, lane, pk, layout == 0 ? kRefSort : kRouted);
  int lt = 0, eq = 0;
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) {
    if (c < wk.nch) {  // wave-uniform
      const int kc = wk.key[c];
      lt += __popcll(__ballot(kc >= 0 && kc < key));
      eq += __popcll(__ballot(kc == key));
    }
  }
  if (lane == 0) {
    s_lt[w] = lt;
    s_eq[w] = eq;
  }
  __syncthreads();
  int off = 0, run = 0;
#pragma unroll
  for (int q = 0; q < kPlanNT / 64; ++q) {
    off += s_lt[q];
    run += q < w ? s_eq[q] : 0;
  }
  run += off;
  const uint64_t below = lane ? ((~0ull) >> (64 - lane)) : 0ull;
#pragma unroll
  for (int c = 0; c < kPlanCh; ++c) {
    if (c < wk.nch) {  // wave-uniform
      const bool hit = wk.key[c] == key;
      const uint64_t m = __ballot(hit);
      if (hit) {
        const int64_t i = wk.lo + 64 * c + lane;
        const int pos = run + __popcll(m & below);
        if (layout == 0) {
          for (int k = 0; k < K; ++k) {
            row_slot[pos * K + k] = (int)i * K + k;
            slot_row[i * K + k] = pos * K + k;
          }
        } else {
          row_slot[pos] = (int)i;
          slot_row[i] = pos;
        }
      }
      run += __popcll(m);
    }
  }
  if (threadIdx.x == 0) {
    if (layout == 0) {
      const int chunk = max(1, M / E);  // E equal chunks; rows past E*chunk are never computed
      offsets[key] = min(key * chunk, M);
      if (key == E - 1) offsets[E] = min(E * chunk, M);
    } else {
      offsets[key] = off;
      if (key == E - 1) offsets[E] = M;  // every slot is kept
    }
    if (key == 0) ndrop[0] = 0;
  }
}

// Multi-block path, per grouping: count -> scan -> rank.
// Count: per block of kPlanIB items, counts[key * nblk + b] (key-major, so that the scan reads each key's
// block counts contiguously); the block's keys are loaded before any is counted.  Block 0 zeroes ndrop in
// the first grouping of a plan.
constexpr int kPlanCountNT = 256;
__global__ __launch_bounds__(kPlanCountNT) void k_plan_count(int mode, PlanKeys pk, int64_t M, int nkeys, int nblk,
                                                             int* __restrict__ counts, int* __restrict__ ndrop,
                                                             int zero_ndrop) {
  extern __shared__ int hist[];
  constexpr int PER = kPlanIB / kPlanCountNT;
  const int64_t beg = (int64_t)blockIdx.x * kPlanIB;
  const int64_t end = min(M, beg + kPlanIB);
  const int64_t st = pk.stride(mode);
  const uint8_t* dp = mode == kRouted ? pk.drop : nullptr;
  int64_t e[PER];
  int d[PER], key[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) e[j] = pk.idx[min(beg + j * kPlanCountNT + threadIdx.x, end - 1) * st];
  if (dp) {
#pragma unroll
    for (int j = 0; j < PER; ++j) d[j] = dp[min(beg + j * kPlanCountNT + threadIdx.x, end - 1)];
  } else {
#pragma unroll
    for (int j = 0; j < PER; ++j) d[j] = 0;
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int64_t i = beg + j * kPlanCountNT + threadIdx.x;
    key[j] = i < end ? pk.key(mode, i, e[j], d[j]) : -1;
  }
  for (int q = threadIdx.x; q < nkeys; q += kPlanCountNT) hist[q] = 0;
  if (blockIdx.x == 0 && threadIdx.x == 0 && zero_ndrop) ndrop[0] = 0;
  __syncthreads();
#pragma unroll
  for (int j = 0; j < PER; ++j)
    if (key[j] >= 0) atomicAdd(&hist[key[j]], 1);
  __syncthreads();
  for (int q = threadIdx.x; q < nkeys; q += kPlanCountNT) counts[(int64_t)q * nblk + blockIdx.x] = hist[q];
}

// Scan: one wave per key, base[key * nblk + b] = the key's items in blocks before b, key_tot[key] = its total.
// The block counts are loaded 256 at a time before they are scanned.
__global__ __launch_bounds__(256) void k_plan_scan(const int* __restrict__ counts, int nblk, int nkeys,
                                                   int* __restrict__ base, int* __restrict__ key_tot) {
  const int lane = threadIdx.x & 63;
  const int key = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
  if (key >= nkeys) return;
  const int* c = counts + (int64_t)key * nblk;
  int* bo = base + (int64_t)key * nblk;
  int run = 0;
  for (int b0 = 0; b0 < nblk; b0 += 256) {
    int v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = b0 + 64 * j + lane;
      v[j] = b < nblk ? c[b] : 0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int incl = v[j];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      const int b = b0 + 64 * j + lane;
      if (b < nblk) bo[b] = run + incl - v[j];
      run += __shfl(incl, 63);
    }
  }
  if (lane == 0) key_tot[key] = run;
}

// Rank: one 1024-thread block per kPlanIB items.  The block loads its keys and its column of the block bases,
// forms kb[key] = key offset (exclusive prefix of key_tot; none for CAPACITY, whose ranks are per key) + the
// key's items in earlier blocks in LDS meanwhile, ranks its items inside the block (16-wave grouping) and adds
// kb.  Block 0 (no earlier blocks) writes the layout's offsets; ROUTED pads row_slot past the kept rows with
// -1 (spread over the blocks).  CAPACITY with counts_next: also the block's kept slots per expert, the count
// pass of the ROUTED grouping that follows (same items, same blocks).
// LDS: cnt [nwr * nkeys] + kb [nkeys + 1] + part [1024] + red [16] + hist [E] ints.
constexpr int kPlanKPT = 8;  // keys per thread of a rank block (nkeys <= 8192)
__global__ __launch_bounds__(kPlanNT) void k_plan_rank(int mode, PlanKeys pk, int64_t nitems, int64_t M, int nkeys,
                                                       int nblk, const int* __restrict__ base,
                                                       const int* __restrict__ key_tot, int64_t capacity,
                                                       uint8_t* __restrict__ drop, int* __restrict__ row_slot,
                                                       int* __restrict__ slot_row, int* __restrict__ offsets,
                                                       int* __restrict__ ndrop, int* __restrict__ counts_next) {
  extern __shared__ int lds[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = pk.K, E = pk.E;
  const int nwr = plan_nwr(nkeys), nbits = nbits_of(nkeys);
  int* cnt = lds;
  int* kb = cnt + nwr * nkeys;
  int* part = kb + nkeys + 1;
  int* red = part + kPlanNT;
  int* hist = red + 16;
  const int b = blockIdx.x;
  WaveKeys wk;
  if (w < nwr)
    load_keys(wk, (int64_t)b * kPlanIB, min(nitems, (int64_t)(b + 1) * kPlanIB), nwr, w, lane, pk, mode);
  int bv[kPlanKPT];
#pragma unroll
  for (int j = 0; j < kPlanKPT; ++j) bv[j] = base[(int64_t)min((int)threadIdx.x + j * kPlanNT, nkeys - 1) * nblk + b];
  for (int q = threadIdx.x; q < nwr * nkeys; q += kPlanNT) cnt[q] = 0;
  if (counts_next)
    for (int q = threadIdx.x; q < E; q += kPlanNT) hist[q] = 0;
  if (mode == kCapacity) __syncthreads();
  else block_excl_scan(key_tot, nkeys, kb, part);  // ends with a barrier
#pragma unroll
  for (int j = 0; j < kPlanKPT; ++j) {
    const int key = threadIdx.x + j * kPlanNT;
    if (key < nkeys) kb[key] = (mode == kCapacity ? 0 : kb[key]) + bv[j];
  }
  if (w < nwr) group_count(wk, w, lane, nkeys, nbits, cnt);
  __syncthreads();
  group_prefix(nwr, nkeys, cnt, nullptr);
  __syncthreads();  // cnt prefixed, kb complete
  if (mode == kCapacity) {
    int dropped = 0;
    if (w < nwr)
      group_rank(wk, w, lane, nkeys, nbits, cnt,
                 [&](int64_t i, int key, int rank) {
                   const bool d = (int64_t)(kb[key] + rank) >= capacity;
                   drop[i] = d ? 1 : 0;
                   dropped += d ? 1 : 0;
                   if (counts_next && !d) atomicAdd(&hist[key % E], 1);
                 },
                 [](int64_t) {});
    const int t = block_sum(dropped, red);  // its barriers also complete the hist updates
    if (threadIdx.x == 0 && t) atomicAdd(ndrop, t);
    if (counts_next)
      for (int q = threadIdx.x; q < E; q += kPlanNT) counts_next[(int64_t)q * nblk + b] = hist[q];
  } else if (mode == kRefSort) {
    const RefOut ro{K, row_slot, slot_row};
    if (w < nwr)
      group_rank(wk, w, lane, nkeys, nbits, cnt, [&](int64_t t, int key, int rank) { ro(t, (int64_t)kb[key] + rank); },
                 [](int64_t) {});
    if (b == 0) {
      const int64_t chunk = max((int64_t)1, M / E);  // E equal chunks; rows past E*chunk are never computed
      for (int e = threadIdx.x; e <= E; e += kPlanNT) offsets[e] = (int)min((int64_t)e * chunk, M);
    }
  } else {
    if (w < nwr)
      group_rank(wk, w, lane, nkeys, nbits, cnt,
                 [&](int64_t i, int key, int rank) {
                   const int row = kb[key] + rank;
                   row_slot[row] = (int)i;
                   slot_row[i] = row;
                 },
                 [&](int64_t i) { slot_row[i] = -1; });
    if (b == 0)
      for (int e = threadIdx.x; e <= E; e += kPlanNT) offsets[e] = kb[e];  // block 0: kb = key offsets
    for (int64_t r = kb[E] + (int64_t)b * kPlanNT + threadIdx.x; r < M; r += (int64_t)nblk * kPlanNT)
      row_slot[r] = -1;  // no row past the kept ones
  }
}

// ---------------------------------------------------------------------------
// Fused multi-block path for capacity drops with the routed layout: count -> scan2 -> rank2 (three launches
// instead of the two groupings' five).  Within one capacity key (column k, expert e) the items of block b take
// the consecutive capacity ranks base[key][b] + 0, 1, ..., so the block keeps exactly
// clamp(capacity - base[key][b], 0, count[key][b]) of them: the routed grouping's block counts follow from the
// capacity scan without a rank pass, and one rank pass does both in-block groupings.
// ---------------------------------------------------------------------------
// Scan2: one wave per expert e.  For each block chunk of 256 blocks it loads the block counts of all K keys
// (k, e) (eight keys per round of loads), writes the capacity bases base[key][b] (exclusive prefix over blocks,
// carried across chunks in LDS), sums the kept slots per block over the K keys and writes their exclusive
// prefix over blocks, base_r[e][b]; tot_r[e] = the expert's kept slots.  base_r may be the counts table itself:
// a lane writes base_r[e][b] only after it has loaded every count of expert e's keys in block b.
__global__ __launch_bounds__(256) void k_plan_scan2(const int* counts, int nblk, int K, int E, int64_t capacity,
                                                    int* __restrict__ base, int* base_r, int* __restrict__ tot_r) {
  __shared__ int s_run[4][kPlanMaxK];  // per wave: the running capacity base of each key (k, e)
  const int lane = threadIdx.x & 63, wq = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wq;
  if (e >= E) return;  // wave-uniform; no block barrier below
  for (int k = lane; k < K; k += 64) s_run[wq][k] = 0;
  int run_r = 0;
  for (int b0 = 0; b0 < nblk; b0 += 256) {
    int kept[4] = {0, 0, 0, 0};
    for (int k0 = 0; k0 < K; k0 += 8) {
      int v[8][4];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int b = b0 + 64 * j + lane;
          v[kk][j] = (k0 + kk < K && b < nblk) ? counts[(int64_t)((k0 + kk) * E + e) * nblk + b] : 0;
        }
      // the 32 wave scans of this round are independent of each other (the carries are added after)
      int incl[8][4];
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
#pragma unroll
        for (int j = 0; j < 4; ++j) incl[kk][j] = v[kk][j];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1)
#pragma unroll
        for (int kk = 0; kk < 8; ++kk)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int t = __shfl_up(incl[kk][j], o);
            if (lane >= o) incl[kk][j] += t;
          }
#pragma unroll
      for (int kk = 0; kk < 8; ++kk) {
        if (k0 + kk < K) {  // wave-uniform
          const int key = (k0 + kk) * E + e;
          int run = s_run[wq][k0 + kk];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int b = b0 + 64 * j + lane;
            const int bc = run + incl[kk][j] - v[kk][j];
            if (b < nblk) base[(int64_t)key * nblk + b] = bc;
            kept[j] += (int)min((int64_t)v[kk][j], max((int64_t)0, capacity - (int64_t)bc));
            run += __shfl(incl[kk][j], 63);
          }
          if (lane == 0) s_run[wq][k0 + kk] = run;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      int incl = kept[j];
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(incl, o);
        if (lane >= o) incl += t;
      }
      const int b = b0 + 64 * j + lane;
      if (b < nblk) base_r[(int64_t)e * nblk + b] = run_r + incl - kept[j];
      run_r += __shfl(incl, 63);
    }
  }
  if (lane == 0) tot_r[e] = run_r;
}

// Rank2: one 1024-thread block per kPlanIB slots.  The capacity grouping (keys k*E + e, block bases from scan2)
// gives each slot its capacity rank and so its drop flag and its key in the routed grouping (its expert, or none
// for a dropped slot: kept in registers when both groupings split the items over the same waves, else read back
// from the drop flags, which a block barrier makes visible to the block); a routed row is the expert's offset
// (exclusive prefix of tot_r) plus the expert's kept slots in earlier blocks plus the in-block rank.  Block 0
// writes the offsets; rows past the kept ones get -1.
// LDS: ccnt [cnw * K*E] + kb [K*E] + cnt [nwr * E] + kbr [E + 1] + part [1024] + red [16] ints.
__global__ __launch_bounds__(kPlanNT) void k_plan_rank2(PlanKeys pk, int64_t M, int nblk, const int* __restrict__ base,
                                                        const int* __restrict__ base_r, const int* __restrict__ tot_r,
                                                        int64_t capacity, uint8_t* drop,
                                                        int* __restrict__ row_slot, int* __restrict__ slot_row,
                                                        int* __restrict__ offsets, int* __restrict__ ndrop) {
  // `drop` is not restrict-qualified: when the two groupings split the block differently the routed pass reads
  // the flags written here back through pk.drop, the same bytes
  extern __shared__ int lds[];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int K = pk.K, E = pk.E;
  const int cnk = K * E, cnw = plan_nwr(cnk), cnb = nbits_of(cnk);
  const int nwr = plan_nwr(E), nbits = nbits_of(E);
  int* ccnt = lds;
  int* kb = ccnt + cnw * cnk;
  int* cnt = kb + cnk;
  int* kbr = cnt + nwr * E;
  int* part = kbr + E + 1;
  int* red = part + kPlanNT;
  const int b = blockIdx.x;
  const int64_t beg = (int64_t)b * kPlanIB, end = min(M, beg + kPlanIB);
  WaveKeys wk;
  if (w < cnw) load_keys(wk, beg, end, cnw, w, lane, pk, kCapacity);
  int bv[kPlanKPT];
#pragma unroll
  for (int j = 0; j < kPlanKPT; ++j) bv[j] = base[(int64_t)min((int)threadIdx.x + j * kPlanNT, cnk - 1) * nblk + b];
  for (int q = threadIdx.x; q < cnw * cnk; q += kPlanNT) ccnt[q] = 0;
  for (int q = threadIdx.x; q < nwr * E; q += kPlanNT) cnt[q] = 0;
  block_excl_scan(tot_r, E, kbr, part);  // kbr = expert offsets; ends with a barrier
#pragma unroll
  for (int j = 0; j < kPlanKPT; ++j) {
    const int key = threadIdx.x + j * kPlanNT;
    if (key < cnk) kb[key] = bv[j];
  }
  if (b == 0)
    for (int e = threadIdx.x; e <= E; e += kPlanNT) offsets[e] = kbr[e];
  if (w < cnw) group_count(wk, w, lane, cnk, cnb, ccnt);
  __syncthreads();  // counts complete, kb and offsets written
  group_prefix(cnw, cnk, ccnt, nullptr);
  for (int e = threadIdx.x; e < E; e += kPlanNT) kbr[e] += base_r[(int64_t)e * nblk + b];
  __syncthreads();
  int dropped = 0;
  // the routed grouping's keys: with the same wave split (nwr == cnw) each kept slot's expert replaces its
  // capacity key in registers (-1 for a dropped slot); otherwise they are read back from the drop flags
  const bool same_split = nwr == cnw;
  if (w < cnw) {
    if (same_split) {
      group_rank_rekey(wk, w, lane, cnk, cnb, ccnt, [&](int64_t i, int key, int rank) {
        const bool d = (int64_t)(kb[key] + rank) >= capacity;
        drop[i] = d ? 1 : 0;
        dropped += d ? 1 : 0;
        return d ? -1 : key % E;
      });
    } else {
      group_rank(wk, w, lane, cnk, cnb, ccnt,
                 [&](int64_t i, int key, int rank) {
                   const bool d = (int64_t)(kb[key] + rank) >= capacity;
                   drop[i] = d ? 1 : 0;
                   dropped += d ? 1 : 0;
                 },
                 [](int64_t) {});
    }
  }
  const int t = block_sum(dropped, red);  // its barriers also make the block's drop flags visible to the block
  if (threadIdx.x == 0 && t) atomicAdd(ndrop, t);
  // the routed grouping of the kept slots
  if (!same_split && w < nwr) load_keys(wk, beg, end, nwr, w, lane, pk, kRouted);
  if (w < nwr) group_count(wk, w, lane, E, nbits, cnt);
  __syncthreads();
  group_prefix(nwr, E, cnt, nullptr);
  __syncthreads();
  if (w < nwr)
    group_rank(wk, w, lane, E, nbits, cnt,
               [&](int64_t i, int key, int rank) {
                 const int row = kbr[key] + rank;  // < kbr[E] <= M (the guard only bounds the store)
                 if (row < M) row_slot[row] = (int)i;
                 slot_row[i] = row;
               },
               [&](int64_t i) { slot_row[i] = -1; });
  const int kept_total = kbr[E];
  for (int64_t r = kept_total + (int64_t)b * kPlanNT + threadIdx.x; r < M; r += (int64_t)nblk * kPlanNT)
    row_slot[r] = -1;  // no row past the kept ones
}

__global__ void k_fill_i32(int* __restrict__ p, int n, int v) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = v;
}

// ---------------------------------------------------------------------------
// Permute: xp[slot_row[t*K+k], :] = x[t, :] for every slot with a computed row (0 <= row < offsets[E]).
// One wave per token: the row is read once, in segments of up to 64 * NCH 16-byte chunks held in registers,
// and written to each of the token's rows (rows of one token lie in different expert segments, so a
// gather by row would read the token K times).  Streaming (non-temporal) stores; the rows are written once.
// ---------------------------------------------------------------------------
template <int NCH>
__global__ __launch_bounds__(256) void k_permute(const uint8_t* __restrict__ x, const int* __restrict__ slot_row,
                                                 const int* __restrict__ offsets, int E, int K, int64_t N,
                                                 int64_t row_bytes, uint8_t* __restrict__ xp) {
  const int lane = threadIdx.x & 63;
  const int live = offsets[E];
  const int64_t nv = row_bytes / 16;
  for (int64_t t = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); t < N;
       t += (int64_t)gridDim.x * 4) {
    const u32x4* src = reinterpret_cast<const u32x4*>(x + t * row_bytes);
    for (int64_t c0 = 0; c0 < nv; c0 += 64 * NCH) {
      u32x4 v[NCH];
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int64_t c = c0 + lane + 64 * j;
        v[j] = c < nv ? __builtin_nontemporal_load(src + c) : u32x4{0u, 0u, 0u, 0u};
      }
      for (int kw = 0; kw < K; kw += 64) {
        const int kn = min(K - kw, 64);
        const int mine = lane < kn ? slot_row[t * K + kw + lane] : -1;
        for (int k = 0; k < kn; ++k) {
          const int r = __builtin_amdgcn_readlane(mine, k);
          if (r < 0 || r >= live) continue;
          u32x4* dst = reinterpret_cast<u32x4*>(xp + (int64_t)r * row_bytes);
#pragma unroll
          for (int j = 0; j < NCH; ++j) {
            const int64_t c = c0 + lane + 64 * j;
            if (c < nv) __builtin_nontemporal_store(v[j], dst + c);
          }
        }
      }
    }
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
  size_t off_counts, off_base, off_keytot, total;
};

// Block tables of the multi-block path (plans the single-block planner does not take; those need none).
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
  p.off_keytot = off;
  off += al256((size_t)(p.nkeys_max + 1) * 4);
  p.total = off;
  return p;
}

// Dynamic LDS above the default 64 KB needs the kernel's attribute raised (once per kernel and size; every
// device the library runs on gets the same value, so the largest size set so far covers the call).
template <typename Kern>
int plan_allow_lds(Kern kernel, size_t bytes, std::atomic<size_t>& set_so_far) {
  if (bytes <= 64 * 1024 || bytes <= set_so_far.load()) return 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          (int)bytes) != hipSuccess)
    return check_launch("moe_plan: hipFuncSetAttribute");
  size_t cur = set_so_far.load();
  while (cur < bytes && !set_so_far.compare_exchange_weak(cur, bytes)) {
  }
  return 0;
}
std::atomic<size_t> g_lds_small{0}, g_lds_rank{0}, g_lds_rank2{0};

// The grouping passes of the multi-block path.  `counted`: the counts table already holds this grouping's
// block counts (written by the capacity rank pass before it).
struct Grouping {
  hipStream_t s;
  const PlanKeys& pk;
  int64_t M;
  const PlanWs& p;
  char* ws;
  uint8_t* drop;
  int *row_slot, *slot_row, *offsets, *ndrop;

  int run(int mode, int64_t nitems, int nkeys, int64_t capacity, bool zero_ndrop, bool counted,
          bool emit_next) const {
    const int nblk = (int)((nitems + kPlanIB - 1) / kPlanIB);
    int* counts = reinterpret_cast<int*>(ws + p.off_counts);
    int* base = reinterpret_cast<int*>(ws + p.off_base);
    int* key_tot = reinterpret_cast<int*>(ws + p.off_keytot);
    if (!counted)
      MOE_LAUNCH("k_plan_count", k_plan_count, dim3(nblk), dim3(kPlanCountNT), (size_t)nkeys * 4, s, mode, pk,
                 nitems, nkeys, nblk, counts, ndrop, zero_ndrop ? 1 : 0);
    MOE_LAUNCH("k_plan_scan", k_plan_scan, dim3((nkeys + 3) / 4), dim3(256), 0, s, counts, nblk, nkeys, base,
               key_tot);
    const size_t lds_rank = (size_t)(plan_nwr(nkeys) * nkeys + nkeys + 1 + kPlanNT + 16 + pk.E) * 4;
    if (int rc = plan_allow_lds(k_plan_rank, lds_rank, g_lds_rank)) return rc;
    // the rank pass of the capacity grouping writes the next grouping's counts over its own (already scanned)
    MOE_LAUNCH("k_plan_rank", k_plan_rank, dim3(nblk), dim3(kPlanNT), lds_rank, s, mode, pk, nitems, M, nkeys, nblk,
               base, key_tot, capacity, drop, row_slot, slot_row, offsets, ndrop, emit_next ? counts : nullptr);
    return check_launch("moe_plan grouping");
  }
};

// LDS of k_plan_rank2 (bytes).
size_t plan_rank2_lds(int K, int E) {
  const int cnk = K * E;
  return (size_t)(plan_nwr(cnk) * cnk + cnk + plan_nwr(E) * E + E + 1 + kPlanNT + 16) * 4;
}

// Capacity drops with the routed layout in three launches (count, scan2, rank2) when the top-k and the rank
// block's LDS allow it.
bool plan_fused_ok(int64_t K, int64_t E) { return K <= kPlanMaxK && plan_rank2_lds((int)K, (int)E) <= 160 * 1024; }

int plan_fused(hipStream_t s, const PlanKeys& pk, int64_t M, const PlanWs& p, char* ws, int64_t capacity,
               uint8_t* drop, int* row_slot, int* slot_row, int* offsets, int* ndrop) {
  const int K = pk.K, E = pk.E, nkeys = K * E;
  const int nblk = (int)((M + kPlanIB - 1) / kPlanIB);
  int* counts = reinterpret_cast<int*>(ws + p.off_counts);
  int* base = reinterpret_cast<int*>(ws + p.off_base);
  int* tot_r = reinterpret_cast<int*>(ws + p.off_keytot);
  // the routed block bases [E][nblk] overwrite the block counts of the keys (0, e), which scan2's wave for
  // expert e reads (and no other wave reads) before it writes them
  int* base_r = counts;
  MOE_LAUNCH("k_plan_count", k_plan_count, dim3(nblk), dim3(kPlanCountNT), (size_t)nkeys * 4, s, kCapacity, pk, M,
             nkeys, nblk, counts, ndrop, 1);
  MOE_LAUNCH("k_plan_scan2", k_plan_scan2, dim3((E + 3) / 4), dim3(256), 0, s, counts, nblk, K, E, capacity, base,
             base_r, tot_r);
  const size_t lds = plan_rank2_lds(K, E);
  if (int rc = plan_allow_lds(k_plan_rank2, lds, g_lds_rank2)) return rc;
  const PlanKeys pkr{pk.idx, drop, K, E};
  MOE_LAUNCH("k_plan_rank2", k_plan_rank2, dim3(nblk), dim3(kPlanNT), lds, s, pkr, M, nblk, base, base_r, tot_r,
             capacity, drop, row_slot, slot_row, offsets, ndrop);
  return check_launch("moe_plan fused");
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

// The plan proper.  Small plans (plan_small_ok): one block does everything in LDS.  Beyond: count / scan /
// rank kernels per grouping with their block tables in `ws` (plan_ws(N, K, E).total bytes; every table is
// written before it is read, so ws needs no initialisation).
int plan_run(const int64_t* idx, int64_t N, int64_t K, int64_t E, int64_t capacity, int layout, uint8_t* drop_out,
             int32_t* row_slot, int32_t* slot_row, int32_t* offsets, int32_t* ndrop, char* ws, hipStream_t s) {
  const int64_t M = N * K;
  uint8_t* drop = capacity >= 0 ? drop_out : nullptr;
  const PlanKeys pk{idx, drop, (int)K, (int)E};
  if (!drop && E <= kPlanByKey && M <= kPlanSmall) {
    MOE_LAUNCH("k_plan_bykey", k_plan_bykey, dim3((unsigned)E), dim3(kPlanNT), 0, s, idx, (int)N, (int)K, (int)E,
               layout, row_slot, slot_row, offsets, ndrop);
    return check_launch("moe_plan");
  }
  if (plan_small_ok(M, (int)K, (int)E, drop != nullptr)) {
    const size_t lds = (size_t)plan_small_lds_ints(M, (int)K, (int)E, drop != nullptr) * 4;
    if (int rc = plan_allow_lds(k_plan_small, lds, g_lds_small)) return rc;
    MOE_LAUNCH("k_plan_small", k_plan_small, dim3(1), dim3(kPlanNT), lds, s, idx, (int)N, (int)K, (int)E, capacity,
               layout, drop, row_slot, slot_row, offsets, ndrop);
    return check_launch("moe_plan");
  }
  const PlanWs p = plan_ws(N, K, E);
  if (drop && layout == 1 && plan_fused_ok(K, E))
    return plan_fused(s, pk, M, p, ws, capacity, drop, row_slot, slot_row, offsets, ndrop);
  const Grouping g{s, pk, M, p, ws, drop, row_slot, slot_row, offsets, ndrop};
  if (drop) {
    // capacity drops; for the routed layout the same pass counts the kept slots per expert and block
    if (int rc = g.run(kCapacity, M, (int)(K * E), capacity, true, false, layout == 1)) return rc;
    if (layout == 0) return g.run(kRefSort, N, (int)E, -1, false, false, false);
    return g.run(kRouted, M, (int)E, -1, false, true, false);
  }
  if (layout == 0) return g.run(kRefSort, N, (int)E, -1, true, false, false);
  return g.run(kRouted, M, (int)E, -1, true, false, false);
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

extern "C" int moe_permute(const void* x, int64_t row_bytes, const int32_t* slot_row, const int32_t* offsets,
                           int64_t N, int64_t K, int64_t E, void* xp, void* stream) {
  if (row_bytes <= 0 || row_bytes % 16 || E < 1 || K < 1 || N < 0)
    return fail_arg("moe_permute: bad arguments (row_bytes must be a positive multiple of 16)");
  if (N == 0) return 0;
  if (!x || !slot_row || !offsets || !xp || !al16(x) || !al16(xp))
    return fail_arg("moe_permute: null or misaligned pointer");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const unsigned nb = (unsigned)std::min<int64_t>(8192, (N + 3) / 4);
  const uint8_t* xb = static_cast<const uint8_t*>(x);
  uint8_t* xpb = static_cast<uint8_t*>(xp);
  // chunks a lane keeps: the whole row in one segment up to 8 KB (H = 4096 in bf16), 8 KB segments beyond
  if (row_bytes <= 4 * 1024)
    MOE_LAUNCH("k_permute", k_permute<4>, dim3(nb), dim3(256), 0, s, xb, slot_row, offsets, (int)E, (int)K, N,
               row_bytes, xpb);
  else
    MOE_LAUNCH("k_permute", k_permute<8>, dim3(nb), dim3(256), 0, s, xb, slot_row, offsets, (int)E, (int)K, N,
               row_bytes, xpb);
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
