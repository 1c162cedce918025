// Grouped SwiGLU expert GEMMs for gfx950 (bf16 in, fp32 accumulate).
//
// One kernel template covers the six products of the expert FFN forward and
// backward.  Each computes C[m, n] = sum_k A[m, k] B[n, k] on
// v_mfma_f32_32x32x16_bf16 with 256x256 block tiles and a 2-stage LDS ring
// (128 KB) of 64-wide k slices, in one of two forms:
//   8 waves of 128x64, the ring filled by LDS-DMA (global_load_lds_dwordx4) so
//     no operand passes through VGPRs (the backward products, whose operands
//     are read with transposing LDS reads);
//   4 waves of 128x128, one per SIMD (the forward products, bf16 and fp8): a third
//     fewer LDS fragment bytes per MFMA; the refill goes through registers two
//     slices ahead, one 16-byte piece at a time between the MFMAs, with every
//     MFMA slot of a k quarter carrying at most one fragment read and one
//     refill piece (described at the loop).  A 64-wide
// slice makes every row of a k-contiguous operand one whole 128-byte line:
// each DMA instruction fetches 8 full lines, which moves about 1.5x the bytes
// per cycle of half-line (32-wide) slices through the CU's load path, the
// path that bounds this kernel.  The refill of a slice is issued as soon as
// every wave has read it and has a whole slice of MFMAs to land; the LDS
// reads of each 16-wide k quarter overlap the MFMAs of the previous one, with
// one workgroup barrier per slice.  Blocks are numbered so that each XCD
// (blockIdx mod 8) runs a contiguous range of logical tiles: tiles that share
// a weight panel stay in one L2.
//
//   operand mode 0 ("rows"): element (i, k) at P[i*ld + k]  (k contiguous);
//                            MFMA fragments are 16-byte LDS reads
//   operand mode 1 ("cols"): element (i, k) at P[k*ld + i]  (i contiguous);
//                            the tile keeps that layout in LDS and fragments are
//                            read with the transposing ds_read_b64_tr_b16
//   GROUP 0 (row-grouped): M = rows of one expert's segment
//            [offsets[e], offsets[e+1]); B is that expert's weight.  Tiles are
//            enumerated from a per-expert tile prefix so imbalanced segments
//            cost only their own tiles.
//   GROUP 1 (k-grouped):   the reduction runs over one expert's rows; C is that
//            expert's weight gradient (experts without rows get zeros).
//   EPI 0  store C (bf16)
//   EPI 1  SwiGLU forward: the B tile interleaves 32 gate rows and the matching
//          32 up rows, so a lane holds g and u of the same (row, f): stores
//          act = silu(g) * u and the pre-activations hgu = [g | u]
//   EPI 2  SwiGLU backward: C = dA; reads hgu and stores dh = [dg | du]
//          with dg = dA u silu'(g), du = dA silu(g).
//   operand mode 2 (both operands, "rows fp8"): e4m3 bytes, k contiguous, with fp32 scales per A row
//          (sa) and per B row (sb, sb2 for the up rows of EPI1).  The host passes K and the leading
//          dimensions in 16-bit units (two fp8 per unit), so the DMA and the LDS tile are byte-for-byte
//          those of a bf16 rows tile: a 64-unit slice holds 128 fp8 k.  Each k step of 64 uses
//          v_mfma_scale_f32_32x32x64_f8f6f4 on 32-byte fragments made of two 16-byte reads (A and B
//          use the same k-to-lane map, which is all the product needs), and the epilogue multiplies by
//          sa[row] * sb[col] before rounding.  The gate/up product (EPI1) writes act block-quantized
//          (e4m3 plus an E8M0 scale per 32 values, aq / aqs), and the down projection passes those
//          block scales to the MFMA (mxs; its sa is then 1).
//
// products (R = rows, per expert e):
//   fwd1  [act | hgu] = xp  . [Wg_e ; Wu_e]^T      A rows(xp), B rows(W),  G0, EPI1
//   fwd2  y           = act . Wd_e^T               A rows,     B rows,     G0, EPI0
//   dA    dh          = dy  . Wd_e  (+ epilogue)   A rows,     B cols(Wd), G0, EPI2
//   dxp   dxp         = dh  . [Wg_e ; Wu_e]        A rows,     B cols(W),  G0, EPI0
//   dWd   dWd_e       = dy_e^T . act_e             A cols,     B cols,     G1, EPI0
//   dW1   [dWg_e;dWu_e] = dh_e^T . xp_e            A cols,     B cols,     G1, EPI0
#include <algorithm>
#include <utility>

#include "common.h"

namespace moe {

struct GemmArgs {
  const uint16_t* A;   // A operand source
  int64_t lda;
  const uint16_t* B;   // B operand source (first half when b_split > 0)
  const uint16_t* B2;  // second B source: B index >= b_split (k for cols mode) / up rows (EPI1)
  int64_t ldb;
  int64_t b_estride;   // per-expert stride of B / B2 (row-grouped), 0 otherwise
  int b_split;
  uint16_t* C;         // output (first half when c_split > 0)
  uint16_t* C2;        // second output: hgu (EPI1), rows >= c_split (k-grouped)
  int64_t ldc;
  int64_t c_estride;   // per-expert stride of C / C2 (k-grouped)
  int c_split;
  const uint16_t* X;   // EPI2: hgu
  int F;               // EPI1 / EPI2: ffn width
  const int* offsets;  // [E+1] row segments
  const int* tile_off; // [E+1] m-tile prefix (row-grouped, computed with this kernel's BM)
  const int* korder;   // [E] expert order of the k-grouped tiles (heaviest first per XCD range)
  const float* sa;     // mode 2: scale of each A row [rows]
  const float* sb;     // mode 2: scale of each B row [E][N] (EPI1: gate rows [E][F])
  const float* sb2;    // mode 2, EPI1: scale of the up rows [E][F]
  uint8_t* aq;         // mode 2, EPI1: act block-quantized (e4m3 [rows][F]) ...
  uint8_t* aqs;        // ... and its E8M0 block scales, slice-major: [(f / 128) * srows + row] * 4 + (f / 32) % 4
  const uint8_t* mxs;  // mode 2, EPI0: the A operand's E8M0 block scales in that layout (A's rows are act's)
  int64_t srows;       // rows per slice of the block-scale layout (a multiple of 4)
  int E;
  int M, N, K;         // k-grouped: M, N fixed; row-grouped: N, K fixed
};

constexpr int GBM = 256, GBN = 256, GBK = 64;
constexpr int GUNITS = 4;                 // LDS ring of operand tiles (unit 2s = A of stage s, 2s+1 = B)
// Wave layouts (template parameter NW): 8 waves of 128x64 (2 x 4, two waves per SIMD) or 4 waves of
// 128x128 (2 x 2, one wave per SIMD with up to 512 registers: a third fewer LDS bytes per MFMA).
constexpr int GWM = 128;
constexpr int GOPB = GBM * GBK * 2;       // bytes of one operand tile per stage (32 KB): one ring unit
constexpr int GCP = GBN + 8;              // epilogue C tile pitch (elements)
constexpr int GSMEM = (GUNITS * GOPB > GBM * GCP * 2) ? GUNITS * GOPB : GBM * GCP * 2;
constexpr int GSCALE = 2 * 256 * 4;       // mode 2: the tile's row and column scales, after the C tile

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(lds_void_t*)p; }
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// 16 zero bytes: the source of every DMA lane whose element lies past the reduction length.
__device__ __attribute__((aligned(16))) const uint16_t g_zero16[8] = {0, 0, 0, 0, 0, 0, 0, 0};

// sigmoid(g) = 1 / (1 + e^-g) with the hardware reciprocal (~1 ulp of fp32; the results are rounded to bf16).
__device__ __forceinline__ float sigmoid_f(float g) { return __builtin_amdgcn_rcpf(1.f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_f(g); }

// s_waitcnt vmcnt(n) (expcnt / lgkmcnt left unconstrained), gfx9 encoding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One LDS-DMA instruction: lane l copies 16 bytes from src into LDS bytes [lds + 16 l, lds + 16 l + 16).
// Issued from asm on purpose: the compiler tracks the builtin's LDS write and then makes every
// LDS read it cannot disambiguate (the transposing reads below) wait for all DMA in flight
// (vmcnt(0)), which would drain the ring each stage.  Completion is ordered by the explicit
// vmcnt waits of the main loop instead.  (m0 is written by SALU and read by the DMA: one wait state.)
__device__ __forceinline__ void lds_dma16(const void* src, uint32_t lds) {
  __asm__ volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds) : "memory");
}


// s_waitcnt vmcnt(n) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void wait_vmcnt_lgkm0() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Workgroup barrier without the vmcnt(0) drain __syncthreads implies (LDS-DMA stays in flight);
// the empty asm statements keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
  __asm__ volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __asm__ volatile("" ::: "memory");
}

// Scheduling pattern for the machine scheduler: NM slots of one MFMA each.  The ND LDS reads of the
// next k half are spread over the first NR slots (early, so their latency hides behind the later
// MFMAs) and the NV LDS-DMA refills take one slot each at the end.
template <int I, int NM, int NR, int ND, int NV>
struct Interleave {
  static __device__ __forceinline__ void run() {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    if constexpr (I < NR) {
      constexpr int nd = ND * (I + 1) / NR - ND * I / NR;
      if constexpr (nd > 0) __builtin_amdgcn_sched_group_barrier(0x100, nd, 0);  // DS read
    }
    if constexpr (I >= NM - NV) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    if constexpr (I + 1 < NM) Interleave<I + 1, NM, NR, ND, NV>::run();
  }
};

// LDS tile layouts (per operand, per stage), both fed by LDS-DMA (lane l of a wave
// instruction writes bytes [16l, 16l+16) of a 1 KB block):
//   rows tile  [256 i][64 k]: row i is 128 bytes = 8 chunks of 8 k; chunk c sits in slot
//              c ^ ((i >> 1) & 7)  -> the 16 rows one 16-lane group of a fragment read
//              touches (same chunk) land in 16 distinct 16-byte bank groups.
//   cols tile  [64 k][256 i]: row k is 512 bytes = 32 chunks of 8 i; chunk c sits in slot
//              c ^ ((k & 3) << 2)  -> the four k-rows a transposing read touches fall in
//              four disjoint 64-byte bank groups.
__device__ __forceinline__ int rows_off(int i, int c) { return i * 128 + ((c ^ ((i >> 1) & 7)) << 4); }
__device__ __forceinline__ int cols_off(int k, int i) { return k * 512 + (((i >> 3) ^ ((k & 3) << 2)) << 4) + ((i & 7) << 1); }

// Fragment (8 bf16) of a 32x32x16 MFMA operand: element j of lane l is (i = base + l%32, k = ks*16 + (l/32)*8 + j).
__device__ __forceinline__ i16x8 frag_rows(const uint8_t* t, int base, int ks, int lane) {
  const int i = base + (lane & 31);
  return *reinterpret_cast<const i16x8*>(t + rows_off(i, ks * 2 + (lane >> 5)));
}
// Same fragment from a cols tile with two ds_read_b64_tr_b16: lane s of each 16-lane group
// addresses (k0 + s/4, i0 + 4*(s%4)) and receives k0..k0+3 of column i0 + s.
__device__ __forceinline__ i16x8 frag_cols(const uint8_t* t, int base, int ks, int lane) {
  const int s = lane & 15;
  const int i = base + 16 * ((lane >> 4) & 1) + 4 * (s & 3);
  const int k = ks * 16 + (lane >> 5) * 8 + (s >> 2);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(t + cols_off(k, i)));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(t + cols_off(k + 4, i)));
  return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

typedef int i32x8 __attribute__((ext_vector_type(8)));
// fp8 operand of a 32x32x64 MFMA k step s of a rows tile: the 16-byte chunks 4s + h and 4s + 2 + h of row
// base + l%32 (h = l/32), i.e. the bf16 fragments of quarters 2s and 2s+1.
__device__ __forceinline__ i32x8 frag_rows_f8(const uint8_t* t, int base, int s, int lane) {
  const u32x4 lo = __builtin_bit_cast(u32x4, frag_rows(t, base, 2 * s, lane));
  const u32x4 hi = __builtin_bit_cast(u32x4, frag_rows(t, base, 2 * s + 1, lane));
  return i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
}
// e4m3 x e4m3 -> fp32 (block scales 127 = 1.0: the per-row / per-column scales are applied in the epilogue).
// With E8M0 block scales the instruction takes k as two blocks of 32 (k 0-31, 32-63 of the step): the first 16
// bytes of every lane's operand lie in block 0 and the last 16 in block 1 (the layout frag_rows_f8 builds:
// chunks 4s + h and 4s + 2 + h), lane i (< 32) supplies row i's scale of block 0 and lane i + 32 row i's scale of
// block 1 (checked on the GPU with one-hot scale patterns).
__device__ __forceinline__ f32x16 mfma32x32x64_f8(const i32x8& a, const i32x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}
// Smallest e with amax <= 448 * 2^e (448 = 0.875 * 2^9), clamped to [-127, 127]; -127 for amax == 0.
__device__ __forceinline__ int mx_exponent(float amax) {
  if (!(amax > 0.f)) return -127;
  int p;
  const float m = frexpf(amax, &p);
  const int e = m <= 0.875f ? p - 9 : p - 8;
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

template <int AMODE, int BMODE, int GROUP, int EPI, int NW>
__global__ __launch_bounds__(NW * 64, 1) void k_gemm(GemmArgs g) {
  constexpr int GNT = NW * 64;
  constexpr int GWN = NW == 8 ? 64 : 128;
  constexpr int QPW = (GOPB / 1024) / NW;  // LDS-DMA instructions per wave per operand per stage
  constexpr int GDMA = 2 * QPW;            // ... for both operands
  constexpr int NW_N = GBN / GWN;
  constexpr int MI = GWM / 32, NI = GWN / 32;
  constexpr bool F8 = AMODE == 2;
  // fp8 down projection: A (act) carries E8M0 block scales, staged per slice beside the ring (2 x 2 KB)
  constexpr bool MX = F8 && EPI == 0;
  constexpr int MXSTAGE = 2048;
  static_assert((AMODE == 2) == (BMODE == 2), "fp8 mode applies to both operands");
  __shared__ __attribute__((aligned(16))) uint8_t smem[GSMEM + (F8 ? GSCALE : 0) + (MX ? 2 * MXSTAGE : 0)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: LDS-DMA targets stay scalar
  const int wm0 = (wv / NW_N) * GWM;
  const int wn0 = (wv % NW_N) * GWN;

  // ---- tile decode: XCD-contiguous logical order over a 1-D grid.  The grid is sized for the most
  // tiles any routing can produce; the real tile count is known only on the device, so it is split
  // into 8 equal contiguous ranges (one per XCD: blockIdx mod 8), and the surplus blocks of every XCD
  // exit at once. ----
  const int xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3);
  int L, e, mbase, mlen, kbase, klen, nt;
  if constexpr (GROUP == 0) {
    const int Tn = (EPI == 1) ? (2 * g.F + GBN - 1) / GBN : (g.N + GBN - 1) / GBN;
    const int total = g.tile_off[g.E] * Tn;
    const int chunk = (total + 7) >> 3;
    L = xcd * chunk + slot;
    if (slot >= chunk || L >= total) return;
    int lo = 0, hi = g.E - 1;  // largest e with tile_off[e] * Tn <= L
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (g.tile_off[mid] * Tn <= L) lo = mid;
      else hi = mid - 1;
    }
    e = lo;
    const int cnt = g.tile_off[e + 1] - g.tile_off[e];
    const int local = L - g.tile_off[e] * Tn;
    nt = local / cnt;
    const int mt = local - nt * cnt;
    mbase = g.offsets[e] + mt * GBM;
    mlen = min(GBM, g.offsets[e + 1] - mbase);
    kbase = 0;
    klen = g.K;
  } else {
    const int Tm = (g.M + GBM - 1) / GBM, Tn = (g.N + GBN - 1) / GBN;
    const int total = g.E * Tm * Tn;
    const int chunk = (total + 7) >> 3;
    L = xcd * chunk + slot;
    if (slot >= chunk || L >= total) return;
    // every expert has Tm * Tn tiles but a reduction as long as its row count: experts are taken in the
    // order korder (dealt to the XCD ranges by decreasing rows, heaviest first within a range), so each
    // XCD gets a similar share of the reduction work and its CUs, which take blocks in order, start on
    // the longest tiles
    const int p = L / (Tm * Tn);
    e = g.korder[p];
    const int r = L - p * Tm * Tn;
    // groups of (up to) 4 m-tiles, n walked within a group: the 32 tiles an XCD runs at once form a
    // 4 x 8 block that shares 12 operand panels per k slice (an n-fastest row of 32 tiles would need 33)
    constexpr int GM = 4;
    const int grp = r / (GM * Tn);
    const int m0 = grp * GM;
    const int gm = min(Tm - m0, GM);
    const int rr = r - grp * GM * Tn;
    const int mt = m0 + rr % gm;
    nt = rr / gm;

    mbase = mt * GBM;
    mlen = min(GBM, g.M - mbase);
    kbase = g.offsets[e];
    klen = g.offsets[e + 1] - kbase;
  }
  const int n0 = nt * GBN;
  const int nlen = (EPI == 1) ? min(GBN, 2 * (g.F - nt * (GBN / 2))) : min(GBN, g.N - n0);
  const int nk = (klen + GBK - 1) / GBK;

  // ---- per-lane DMA sources.  Wave instruction j (= QPW*wv + q, q < QPW) of an operand fills bytes
  // [1024 j, 1024 j + 1024) of its stage tile: rows mode -> rows 8j + l/8, slot l%8 (one whole
  // 128-byte line per row); cols mode -> k-rows 2j + l/32, slot l%32.  Rows / columns past the
  // tile are clamped to valid ones (their results are never stored), so a stage that lies wholly
  // inside the reduction range needs only a wave-uniform step per instruction: rows mode adds k0
  // elements, cols mode k0 * ld. ----
  const uint16_t* a_src[QPW];
  const uint16_t* b_src[QPW];
  const uint16_t* b_src2[QPW];
  int a_kl_[QPW], b_kl_[QPW];  // the lane's first k within a stage
  auto a_kl = [&](int q) { return a_kl_[q]; };
  auto b_kl = [&](int q) { return b_kl_[q]; };
  auto a_at = [&](int q, int64_t step) -> const uint16_t* { return a_src[q] + step; };
  auto b_at = [&](int q, int64_t step) -> const uint16_t* { return b_src[q] + step; };
#pragma unroll
  for (int q = 0; q < QPW; ++q) {
    const int j = QPW * wv + q;
    if constexpr (AMODE != 1) {
      const int i = 8 * j + (lane >> 3);
      a_kl_[q] = ((lane & 7) ^ ((i >> 1) & 7)) * 8;
      a_src[q] = g.A + (int64_t)(mbase + min(i, mlen - 1)) * g.lda + kbase + a_kl_[q];
    } else {
      a_kl_[q] = 2 * j + (lane >> 5);
      const int i = (((lane & 31) ^ ((a_kl_[q] & 3) << 2)) << 3);
      a_src[q] = g.A + (int64_t)(kbase + a_kl_[q]) * g.lda + mbase + (i < mlen ? i : 0);
    }
    b_src2[q] = nullptr;
    if constexpr (BMODE != 1) {
      const int i = 8 * j + (lane >> 3);
      b_kl_[q] = ((lane & 7) ^ ((i >> 1) & 7)) * 8;
      const int ic = min(i, nlen - 1);
      if constexpr (EPI == 1) {
        const int f = nt * (GBN / 2) + (ic >> 6) * 32 + (ic & 31);
        b_src[q] = (((ic >> 5) & 1) ? g.B2 : g.B) + (int64_t)e * g.b_estride + (int64_t)f * g.ldb + b_kl_[q];
      } else {
        b_src[q] = g.B + (int64_t)e * g.b_estride + (int64_t)(n0 + ic) * g.ldb + b_kl_[q];
      }
    } else {
      b_kl_[q] = 2 * j + (lane >> 5);
      int i = (((lane & 31) ^ ((b_kl_[q] & 3) << 2)) << 3);
      i = i < nlen ? i : 0;
      if constexpr (GROUP == 0) {
        b_src[q] = g.B + (int64_t)e * g.b_estride + (int64_t)b_kl_[q] * g.ldb + n0 + i;
        if (g.b_split > 0) b_src2[q] = g.B2 + (int64_t)e * g.b_estride + (int64_t)b_kl_[q] * g.ldb + n0 + i;
      } else {
        b_src[q] = g.B + (int64_t)(kbase + b_kl_[q]) * g.ldb + n0 + i;
      }
    }
  }

  // Refill a ring unit with the A (issue_a) or B (issue_b) tile of k slice kt.  Fast path (a
  // wave-uniform branch): the slice lies inside the reduction range and on one side of b_split.
  // Otherwise each lane checks its own k: past klen it reads 16 zero bytes, and cols-mode B switches
  // to the second source at k = b_split.
  auto issue_a = [&](int kt, uint8_t* unit) {
    const int k0 = kt * GBK;
    uint8_t* const sa = unit + QPW * wv * 1024;
    const int64_t step = AMODE != 1 ? (int64_t)k0 : (int64_t)k0 * g.lda;
    if (k0 + GBK <= klen) {
#pragma unroll
      for (int q = 0; q < QPW; ++q) lds_dma16(a_at(q, step), lds_addr(sa + q * 1024));
    } else {
#pragma unroll
      for (int q = 0; q < QPW; ++q)
        lds_dma16(k0 + a_kl(q) < klen ? a_at(q, step) : g_zero16, lds_addr(sa + q * 1024));
    }
  };
  auto issue_b = [&](int kt, uint8_t* unit) {
    const int k0 = kt * GBK;
    const bool kfull = k0 + GBK <= klen;
    uint8_t* const sb = unit + QPW * wv * 1024;
    const int64_t bld = BMODE != 1 ? 1 : g.ldb;
    bool split = false;
    if constexpr (BMODE == 1 && GROUP == 0) split = g.b_split > 0 && k0 + GBK > g.b_split;
    if (!split) {
      const int64_t step = (int64_t)k0 * bld;
      if (kfull) {
#pragma unroll
        for (int q = 0; q < QPW; ++q) lds_dma16(b_at(q, step), lds_addr(sb + q * 1024));
      } else {
#pragma unroll
        for (int q = 0; q < QPW; ++q)
          lds_dma16(k0 + b_kl(q) < klen ? b_at(q, step) : g_zero16, lds_addr(sb + q * 1024));
      }
    } else {
      const int64_t step1 = (int64_t)k0 * bld, step2 = (int64_t)(k0 - g.b_split) * bld;
      if (kfull && k0 >= g.b_split) {
#pragma unroll
        for (int q = 0; q < QPW; ++q) lds_dma16(b_src2[q] + step2, lds_addr(sb + q * 1024));
      } else {
#pragma unroll
        for (int q = 0; q < QPW; ++q) {
          const int k = k0 + b_kl(q);
          const uint16_t* src = k >= klen ? g_zero16 : (k < g.b_split ? b_src[q] + step1 : b_src2[q] + step2);
          lds_dma16(src, lds_addr(sb + q * 1024));
        }
      }
    }
  };
  // Ring unit u (A of slice u/2 when u is even, B otherwise) lives in LDS slot u % GUNITS.
  auto unit_ptr = [&](int u) { return smem + (u & (GUNITS - 1)) * GOPB; };
  auto issue_unit = [&](int u) {
    if (u & 1) issue_b(u >> 1, unit_ptr(u));
    else issue_a(u >> 1, unit_ptr(u));
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[mi][ni][j] = 0.f;

  // Fragments of one 16-wide k half of a stage, and the MFMAs that consume them.
  auto frags = [&](const uint8_t* as, const uint8_t* bs, int ks, i16x8 (&fa)[MI], i16x8 (&fb)[NI]) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
      fa[mi] = AMODE != 1 ? frag_rows(as, wm0 + mi * 32, ks, lane) : frag_cols(as, wm0 + mi * 32, ks, lane);
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
      fb[ni] = BMODE != 1 ? frag_rows(bs, wn0 + ni * 32, ks, lane) : frag_cols(bs, wn0 + ni * 32, ks, lane);
  };
  auto mma = [&](const i16x8 (&fa)[MI], const i16x8 (&fb)[NI]) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
        acc[mi][ni] = mfma32x32x16(__builtin_bit_cast(bf16x8, fa[mi]), __builtin_bit_cast(bf16x8, fb[ni]), acc[mi][ni]);
  };

  static_assert(!F8 || NW == 4, "the fp8 products run the 4-wave loop");
  if constexpr (NW == 4) {
    static_assert(AMODE == BMODE && AMODE != 1, "the 4-wave main loop takes k-contiguous operands");
    // One wave per SIMD, 128x128 per wave.  The refill goes through registers two slices ahead: while slice
    // kt is computed, each wave writes its share of slice kt+1 (loaded during slice kt-1) into the free LDS
    // slot and loads its share of slice kt+2 into the same registers, one piece (16 bytes a lane) at a time
    // between the MFMAs, so global loads, LDS writes and fragment reads are spread over the slice.  The loads
    // are ordinary global loads through an address_space(1) pointer: the compiler sees each load's destination
    // st[p] and places the vmcnt wait before the LDS write that reads it (piece p of slice kt+1 was loaded NP
    // loads before piece p of slice kt+2, so that wait is vmcnt(NP-1) and leaves the newer loads in flight).
    // The loop has no explicit vmcnt wait of its own; a load issued from asm here would need one.
    constexpr int NP = 2 * QPW;  // pieces per wave per slice: A pieces 0..QPW-1, then B
    u32x4 st[NP];
    // source of piece p of slice kt; `full`: the slice lies inside the reduction range and on one side of
    // b_split (no per-lane check)
    auto gsrc = [&](int kt, int p, bool full) -> const uint16_t* {
      const int k0 = kt * GBK;
      if (p < QPW) {
        const int q = p;
        const int64_t step = AMODE != 1 ? (int64_t)k0 : (int64_t)k0 * g.lda;
        if (full) return a_at(q, step);
        return (k0 + a_kl(q) < klen) ? a_at(q, step) : g_zero16;
      }
      const int q = p - QPW;
      const int64_t bld = BMODE != 1 ? 1 : g.ldb;
      if (full) {
        if constexpr (BMODE == 1 && GROUP == 0) {
          if (g.b_split > 0 && k0 >= g.b_split) return b_src2[q] + (int64_t)(k0 - g.b_split) * bld;
        }
        return b_at(q, (int64_t)k0 * bld);
      }
      const int k = k0 + b_kl(q);
      if (k >= klen) return g_zero16;
      if constexpr (BMODE == 1 && GROUP == 0) {
        if (g.b_split > 0 && k >= g.b_split) return b_src2[q] + (int64_t)(k0 - g.b_split) * bld;
      }
      return b_at(q, (int64_t)k0 * bld);
    };
    auto slice_full = [&](int kt) {
      const int k0 = kt * GBK;
      bool f = k0 + GBK <= klen;
      if constexpr (BMODE == 1 && GROUP == 0) f = f && !(g.b_split > 0 && k0 < g.b_split && k0 + GBK > g.b_split);
      return f;
    };
    typedef __attribute__((address_space(1))) const u32x4 g_u32x4;
    auto gload = [&](int kt, int p, bool full) {
      st[p] = *reinterpret_cast<g_u32x4*>(reinterpret_cast<uintptr_t>(gsrc(kt, p, full)));
    };
    // ring units and tiles as the DMA path lays them out (piece q of wave wv fills bytes [1024 j, 1024 j + 1024),
    // j = QPW wv + q, of its unit)
    auto lwrite = [&](int kt, int p) {
      const int op = p < QPW ? 0 : 1, q = p < QPW ? p : p - QPW;
      __asm__ volatile("" ::: "memory");
      *reinterpret_cast<u32x4*>(unit_ptr(2 * kt + op) + (QPW * wv + q) * 1024 + lane * 16) = st[p];
      __asm__ volatile("" ::: "memory");
    };
    if constexpr (F8) {
      // fp8: each 128-byte k slice is two 64-k steps of MI x NI MFMAs (32x32x64, e4m3).  One fragment set is
      // live: an A fragment is re-read for the next step right after its row's last MFMA of this step, a B
      // fragment after its column's (the last row of MFMAs), so the reads of step s+1 run under the MFMAs of
      // step s without a second set of registers.  The refill pieces of slice kt+1 (LDS writes) and kt+2
      // (global loads) go one per MFMA slot into step 0 and the first half of step 1; then each wave waits
      // for its own LDS traffic, one barrier makes slice kt+1 visible, and the second half of step 1 reads
      // slice kt+1's step-0 fragments as they free up.  With block-scaled A (MX) the slice's scale window (2 KB
      // from the 4-row-aligned row below the tile's first row) rides along as one
      // more piece (512 bytes a wave, lanes 32-63 repeating lanes 0-31) into a 2-slot LDS area, and each lane reads its rows' scale
      // words of slice kt+1 right after that barrier.
      constexpr int NPX = NP + (MX ? 1 : 0);  // pieces per slice, the scale window last
      constexpr int PA = NPX - 8;             // pieces in step 0; the other 8 in step 1's first half
      static_assert(MI * NI == 16 && NI == 4 && PA <= 16, "fp8 4-wave slot plan");
      uint8_t* const mx_lds = smem + GSMEM + GSCALE;
      const int mx_r0 = mbase & 3;
      u32x4 st_mx;
      auto gload_x = [&](int kt, int p, bool full) {
        if constexpr (MX) {
          if (p == NP) {  // lanes 32-63 repeat lanes 0-31 (no divergent branch in the slot sequence)
            st_mx = *reinterpret_cast<g_u32x4*>(reinterpret_cast<uintptr_t>(
                g.mxs + ((int64_t)kt * g.srows + (mbase - mx_r0)) * 4 + (wv * 32 + (lane & 31)) * 16));
            return;
          }
        }
        gload(kt, p, full);
      };
      auto lwrite_x = [&](int kt, int p) {
        if constexpr (MX) {
          if (p == NP) {
            __asm__ volatile("" ::: "memory");
            *reinterpret_cast<u32x4*>(mx_lds + (kt & 1) * MXSTAGE + (wv * 32 + (lane & 31)) * 16) = st_mx;
            __asm__ volatile("" ::: "memory");
            return;
          }
        }
        lwrite(kt, p);
      };
      i32x8 fa[MI], fb[NI];
      int sw[MI];
      uint32_t swn[MI];
      // the lane's scale word of each of its MI rows for slice kt (raw), and the form the MFMA takes: shifted
      // so that byte 2 st of the word is block 2 st + h (lane half h supplies the scale of the step's block h);
      // the shift waits for the read, so it is applied only where the words are taken into use
      auto read_sw = [&](int kt, uint32_t (&w)[MI]) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
          w[mi] = *reinterpret_cast<const uint32_t*>(mx_lds + (kt & 1) * MXSTAGE +
                                                     (mx_r0 + wm0 + mi * 32 + (lane & 31)) * 4);
      };
      auto use_sw = [&](const uint32_t (&w)[MI]) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) sw[mi] = (int)(w[mi] >> (8 * (lane >> 5)));
      };
      // MFMA slots [SLO, SHI) of step ST (slot i = row i / NI, column i % NI); after slot i the next step's
      // fragments that it frees are read from (nas, nbs, step nst) when read_next, and refill piece
      // PLO + (i - SLO) moves when below PHI.  MODE as in the bf16 loop (0: write kt+1 / load full kt+2,
      // 1: load with checks, 2: write only, 3: none).
      auto slots = [&](auto st_c, auto slo_c, auto shi_c, auto mode_c, auto plo_c, auto phi_c, const uint8_t* nas,
                       const uint8_t* nbs, int nst, bool read_next, int kt, bool lfull) {
        constexpr int ST = decltype(st_c)::value, SLO = decltype(slo_c)::value, SHI = decltype(shi_c)::value;
        constexpr int MODE = decltype(mode_c)::value, PLO = decltype(plo_c)::value, PHI = decltype(phi_c)::value;
        [&]<int... I>(std::integer_sequence<int, I...>) {
          (([&] {
             constexpr int i = SLO + I;
             constexpr int mi = i / NI, ni = i % NI;
             if constexpr (MX)
               acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[mi], fb[ni], acc[mi][ni], 0, 0,
                                                                             2 * ST, sw[mi], 0, 127);
             else
               acc[mi][ni] = mfma32x32x64_f8(fa[mi], fb[ni], acc[mi][ni]);
             __builtin_amdgcn_sched_barrier(0);
             if (read_next) {
               if constexpr (ni == NI - 1) fa[mi] = frag_rows_f8(nas, wm0 + mi * 32, nst, lane);
               if constexpr (mi == MI - 1) fb[ni] = frag_rows_f8(nbs, wn0 + ni * 32, nst, lane);
             }
             constexpr int p = PLO + I;
             if constexpr (MODE < 3 && p < PHI) {
               lwrite_x(kt + 1, p);
               if constexpr (MODE == 0) gload_x(kt + 2, p, true);
               else if constexpr (MODE == 1) gload_x(kt + 2, p, lfull);
             }
             __builtin_amdgcn_sched_barrier(0);
           }()), ...);
        }(std::make_integer_sequence<int, SHI - SLO>{});
      };
      using C0 = std::integral_constant<int, 0>;
      using C1 = std::integral_constant<int, 1>;
      using C8 = std::integral_constant<int, 8>;
      using C16 = std::integral_constant<int, 16>;
      using CPA = std::integral_constant<int, PA>;
      using CNP = std::integral_constant<int, NPX>;
      using M3 = std::integral_constant<int, 3>;
      auto slice = [&](auto mode_c, int kt) {
        const uint8_t* const ca = unit_ptr(2 * kt);
        const uint8_t* const cb = unit_ptr(2 * kt + 1);
        const bool lfull = kt + 2 < nk ? slice_full(kt + 2) : true;
        slots(C0{}, C0{}, C16{}, mode_c, C0{}, CPA{}, ca, cb, 1, true, kt, lfull);
        slots(C1{}, C0{}, C8{}, mode_c, CPA{}, CNP{}, ca, cb, 0, false, kt, lfull);
        wait_vmcnt_lgkm0<63>();  // this wave's LDS writes of slice kt+1 and reads of slice kt are done
        lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const bool more = kt + 1 < nk;
        const uint8_t* const na = unit_ptr(2 * kt + 2);
        const uint8_t* const nb = unit_ptr(2 * kt + 3);
        if (more) {
          // rows 0 and 1 finished their MFMAs in the first half of step 1
#pragma unroll
          for (int mi = 0; mi < 8 / NI; ++mi) fa[mi] = frag_rows_f8(na, wm0 + mi * 32, 0, lane);
          if constexpr (MX) read_sw(kt + 1, swn);
        }
        __builtin_amdgcn_sched_barrier(0);
        slots(C1{}, C8{}, C16{}, M3{}, C0{}, C0{}, na, nb, 0, more, kt, true);
        if constexpr (MX) use_sw(swn);
      };
      if (nk > 0) {
        for (int p = 0; p < NPX; ++p) gload_x(0, p, slice_full(0));
        for (int p = 0; p < NPX; ++p) lwrite_x(0, p);
        if (nk > 1) {
          for (int p = 0; p < NPX; ++p) gload_x(1, p, slice_full(1));
        }
        __syncthreads();
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) fa[mi] = frag_rows_f8(unit_ptr(0), wm0 + mi * 32, 0, lane);
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) fb[ni] = frag_rows_f8(unit_ptr(1), wn0 + ni * 32, 0, lane);
        if constexpr (MX) {
          read_sw(0, swn);
          use_sw(swn);
        }
        int kt = 0;
        for (; kt + 3 < nk && slice_full(kt + 2); ++kt) slice(C0{}, kt);
        for (; kt + 2 < nk; ++kt) slice(C1{}, kt);
        if (kt + 1 < nk) slice(std::integral_constant<int, 2>{}, kt++);
        if (kt < nk) slice(M3{}, kt);
      }
    } else {
    auto read_frag = [&](const uint8_t* as, const uint8_t* bs, int ks, int f, i16x8 (&fa)[MI], i16x8 (&fb)[NI]) {
      if (f < MI) fa[f] = frag_rows(as, wm0 + f * 32, ks, lane);
      else fb[f - MI] = frag_rows(bs, wn0 + (f - MI) * 32, ks, lane);
    };
    // One k quarter as 16 MFMA slots (mi-major), each followed by at most one fragment read of the next
    // quarter (slots 0..MI+NI-1) and at most one refill piece (slots 8.., pieces [PLO, PHI)); sched_barrier
    // keeps this order.  MODE 0: steady state (write slice kt+1, load full slice kt+2); 1: write, load with
    // checks; 2: write only (no slice left to load); 3: no refill.
    auto quarter = [&](auto mode_c, auto plo_c, auto phi_c, const i16x8 (&ca)[MI], const i16x8 (&cb)[NI],
                       const uint8_t* nas, const uint8_t* nbs, int nks, bool read_next, i16x8 (&na)[MI],
                       i16x8 (&nb)[NI], int kt, bool lfull) {
      constexpr int MODE = decltype(mode_c)::value;
      constexpr int PLO = decltype(plo_c)::value, PHI = decltype(phi_c)::value;
      [&]<int... I>(std::integer_sequence<int, I...>) {
        (([&] {
           constexpr int i = I;
           constexpr int mi = i / NI, ni = i % NI;
           acc[mi][ni] = mfma32x32x16(__builtin_bit_cast(bf16x8, ca[mi]), __builtin_bit_cast(bf16x8, cb[ni]), acc[mi][ni]);
           __builtin_amdgcn_sched_barrier(0);
           if constexpr (i < MI + NI) {
             if (read_next) read_frag(nas, nbs, nks, i, na, nb);
           }
           constexpr int p = PLO + (i - 8);
           if constexpr (MODE < 3 && i >= 8 && p < PHI) {
             lwrite(kt + 1, p);
             if constexpr (MODE == 0) gload(kt + 2, p, true);
             else if constexpr (MODE == 1) gload(kt + 2, p, lfull);
           }
           __builtin_amdgcn_sched_barrier(0);
         }()), ...);
      }(std::make_integer_sequence<int, MI * NI>{});
    };
    constexpr int PB1 = (NP + 2) / 3, PB2 = (2 * NP + 2) / 3;
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, PB1>;
    using P2 = std::integral_constant<int, PB2>;
    using P3 = std::integral_constant<int, NP>;
    i16x8 fa0[MI], fb0[NI], fa1[MI], fb1[NI];
    auto slice = [&](auto mode_c, int kt) {
      const uint8_t* const ca = unit_ptr(2 * kt);
      const uint8_t* const cb = unit_ptr(2 * kt + 1);
      const bool lfull = kt + 2 < nk ? slice_full(kt + 2) : true;
      quarter(mode_c, P0{}, P1{}, fa0, fb0, ca, cb, 1, true, fa1, fb1, kt, lfull);
      quarter(mode_c, P1{}, P2{}, fa1, fb1, ca, cb, 2, true, fa0, fb0, kt, lfull);
      quarter(mode_c, P2{}, P3{}, fa0, fb0, ca, cb, 3, true, fa1, fb1, kt, lfull);
      wait_vmcnt_lgkm0<63>();  // this wave's LDS writes of slice kt+1 and reads of slice kt are done
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
      quarter(std::integral_constant<int, 3>{}, P3{}, P3{}, fa1, fb1, unit_ptr(2 * kt + 2), unit_ptr(2 * kt + 3), 0,
              kt + 1 < nk, fa0, fb0, kt, true);
    };
    if (nk > 0) {
      for (int p = 0; p < NP; ++p) gload(0, p, slice_full(0));
      for (int p = 0; p < NP; ++p) lwrite(0, p);
      if (nk > 1) {
        for (int p = 0; p < NP; ++p) gload(1, p, slice_full(1));
      }
      __syncthreads();
      frags(unit_ptr(0), unit_ptr(1), 0, fa0, fb0);
      int kt = 0;
      // steady state: slice kt+2 <= nk-2 is full (only the last slice of the reduction can be partial,
      // and b_split falls on a slice boundary whenever every slice is full)
      for (; kt + 3 < nk && slice_full(kt + 2); ++kt) slice(std::integral_constant<int, 0>{}, kt);
      for (; kt + 2 < nk; ++kt) slice(std::integral_constant<int, 1>{}, kt);
      if (kt + 1 < nk) slice(std::integral_constant<int, 2>{}, kt++);
      if (kt < nk) slice(std::integral_constant<int, 3>{}, kt);
    }
    }
    wait_vmcnt<0>();
  } else if (nk > 0) {
    // Software pipeline over the four 16-wide k quarters of a stage: the LDS reads of quarter q+1 are
    // interleaved with the MFMAs of quarter q (register sets 0 and 1 alternate).  Before the last
    // quarter of stage kt every wave waits for stage kt+1 (the only DMA group in flight) and for its
    // own reads of stage kt; one barrier makes both visible workgroup-wide, and stage kt's two units
    // are refilled with stage kt+2 while the last quarter's MFMAs run.
    issue_unit(0);
    issue_unit(1);
    if (nk > 1) {
      issue_unit(2);
      issue_unit(3);
    }
    if (nk > 1) wait_vmcnt<2 * QPW>();  // this wave's part of stage 0 has landed
    else wait_vmcnt<0>();
    lds_barrier();                                   // every wave's part has
    i16x8 fa0[MI], fb0[NI], fa1[MI], fb1[NI];
    frags(unit_ptr(0), unit_ptr(1), 0, fa0, fb0);
    constexpr int NDS = (AMODE ? 2 : 1) * MI + (BMODE ? 2 : 1) * NI;  // LDS read instructions per k quarter
    for (int kt = 0; kt < nk; ++kt) {
      const uint8_t* const ca = unit_ptr(2 * kt);
      const uint8_t* const cb = unit_ptr(2 * kt + 1);
      frags(ca, cb, 1, fa1, fb1);
      mma(fa0, fb0);
      Interleave<0, MI * NI, MI * NI / 2, NDS, 0>::run();
      __builtin_amdgcn_sched_barrier(0);
      frags(ca, cb, 2, fa0, fb0);
      mma(fa1, fb1);
      Interleave<0, MI * NI, MI * NI / 2, NDS, 0>::run();
      __builtin_amdgcn_sched_barrier(0);
      frags(ca, cb, 3, fa1, fb1);
      mma(fa0, fb0);
      Interleave<0, MI * NI, MI * NI / 2, NDS, 0>::run();
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt_lgkm0<0>();  // stage kt+1 landed; this wave's reads of stage kt are done
      lds_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (kt + 2 < nk) {
        issue_unit(2 * kt + 4);
        issue_unit(2 * kt + 5);
      }
      if (kt + 1 < nk) frags(unit_ptr(2 * kt + 2), unit_ptr(2 * kt + 3), 0, fa0, fb0);
      mma(fa1, fb1);
      Interleave<0, MI * NI, MI * NI / 2, NDS, 0>::run();
      __builtin_amdgcn_sched_barrier(0);
    }
    wait_vmcnt<0>();
  }
  __syncthreads();

  // ---- epilogue: the bf16 C tile goes through LDS so every global access is a 16-byte row chunk.
  // acc[mi][ni][j] = C[wm0 + mi*32 + (j/4)*8 + (lane/32)*4 + j%4][wn0 + ni*32 + lane%32]
  constexpr int CP = GCP;
  uint16_t* cs = reinterpret_cast<uint16_t*>(smem);
  if constexpr (F8) {
    // the tile's row scales [256] and column scales [256] (rows / columns past the tile clamped)
    float* s_sc = reinterpret_cast<float*>(smem + GSMEM);
    if (tid < 256) {
      s_sc[tid] = MX ? 1.f : g.sa[mbase + min(tid, mlen - 1)];  // MX: the row scales were applied per block
      float sb;
      if constexpr (EPI == 1) {
        const int f = min(nt * (GBN / 2) + (tid >> 6) * 32 + (tid & 31), g.F - 1);
        sb = (((tid >> 5) & 1) ? g.sb2 : g.sb)[(int64_t)e * g.F + f];
      } else {
        sb = g.sb[(int64_t)e * g.N + min(n0 + tid, g.N - 1)];
      }
      s_sc[256 + tid] = sb;
    }
    __syncthreads();
    if constexpr (EPI == 1) {
      if (g.aq != nullptr && g.C2 == nullptr) {
        // inference: no pre-activations to store, so the SwiGLU runs on the accumulators (a lane holds the gate
        // and the up value of one f in acc[mi][2p][j] and acc[mi][2p + 1][j]: tile columns 64 (c / 64) + c % 32
        // and + 32) with the same roundings as below (gate and up to bf16, act to bf16), and only act goes
        // through LDS, as a [256][128 + 8] bf16 tile, for the block quantization (the same per-chunk code as
        // the general path, reading one 16-byte act chunk instead of the gate and up chunks)
        constexpr int AP = GBN / 2 + 8;
        static_assert(NI == 4, "two gate/up pairs per wave");
        // column scales of the lane's two pairs (gate, up); each row scale is read once for both pairs, and
        // each bf16 rounding converts two values at once (the same rounding as one at a time)
        const int cg0 = wn0 + (lane & 31), cg1 = cg0 + 64;
        const float sg0 = s_sc[256 + cg0], su0 = s_sc[256 + cg0 + 32];
        const float sg1 = s_sc[256 + cg1], su1 = s_sc[256 + cg1 + 32];
        const int fc0 = (cg0 >> 6) * 32 + (lane & 31), fc1 = (cg1 >> 6) * 32 + (lane & 31);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int r = wm0 + mi * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
            const float sr = s_sc[r];
            const uint32_t gu0 = pack2bf(acc[mi][0][j] * sr * sg0, acc[mi][1][j] * sr * su0);
            const uint32_t gu1 = pack2bf(acc[mi][2][j] * sr * sg1, acc[mi][3][j] * sr * su1);
            const uint32_t a01 = pack2bf(silu_f(__uint_as_float(gu0 << 16)) * __uint_as_float(gu0 & 0xffff0000u),
                                         silu_f(__uint_as_float(gu1 << 16)) * __uint_as_float(gu1 & 0xffff0000u));
            cs[r * AP + fc0] = (uint16_t)a01;
            cs[r * AP + fc1] = (uint16_t)(a01 >> 16);
          }
        __syncthreads();
        constexpr int QPR = GBN / 16;  // 8-f chunks per row
        for (int u = tid; u < GBM * QPR; u += GNT) {
          const int r = u / QPR, q = u % QPR;
          const int f = nt * (GBN / 2) + q * 8;
          const bool ok = r < mlen && f < g.F;
          const u32x4 av = *reinterpret_cast<const u32x4*>(&cs[r * AP + q * 8]);
          float a[8];
          float amax = 0.f;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            a[2 * d] = __uint_as_float(av[d] << 16);
            a[2 * d + 1] = __uint_as_float(av[d] & 0xffff0000u);
            amax = fmaxf(amax, fmaxf(fabsf(a[2 * d]), fabsf(a[2 * d + 1])));
          }
          amax = ok ? amax : 0.f;
          amax = fmaxf(amax, __shfl_xor(amax, 1));
          amax = fmaxf(amax, __shfl_xor(amax, 2));
          const int ex = mx_exponent(amax);
          const float sc = ldexpf(1.f, -ex);
          const int64_t row = mbase + r;
          if (ok) {
            int lo = 0, hi = 0;
            lo = __builtin_amdgcn_cvt_pk_fp8_f32(a[0] * sc, a[1] * sc, lo, false);
            lo = __builtin_amdgcn_cvt_pk_fp8_f32(a[2] * sc, a[3] * sc, lo, true);
            hi = __builtin_amdgcn_cvt_pk_fp8_f32(a[4] * sc, a[5] * sc, hi, false);
            hi = __builtin_amdgcn_cvt_pk_fp8_f32(a[6] * sc, a[7] * sc, hi, true);
            *reinterpret_cast<uint2*>(g.aq + row * g.F + f) = uint2{(unsigned)lo, (unsigned)hi};
            if (g.C != nullptr) *reinterpret_cast<u32x4*>(g.C + row * g.ldc + f) = av;
          }
          if (r < mlen && (q & 3) == 0)
            g.aqs[((int64_t)nt * g.srows + row) * 4 + (q >> 2)] = (uint8_t)(f < g.F ? ex + 127 : 127);
        }
        return;
      }
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int c = wn0 + ni * 32 + (lane & 31);
        const float sc = s_sc[256 + c];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int r = wm0 + mi * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
          cs[r * CP + c] = f2bf(acc[mi][ni][j] * s_sc[r] * sc);
        }
      }
  } else {
    if constexpr (EPI == 1) {
      if (g.C2 == nullptr) {
        // inference (no pre-activations to store): act formed on the accumulators as in the fp8 epilogue above
        // (gate and up rounded to bf16, act rounded to bf16), and only act goes through LDS, as a [256][128 + 8]
        // bf16 tile, to leave as 16-byte row chunks
        constexpr int AP = GBN / 2 + 8;
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
#pragma unroll
          for (int pr = 0; pr < NI / 2; ++pr) {
            const int cg = wn0 + 2 * pr * 32 + (lane & 31);
            const int fc = (cg >> 6) * 32 + (lane & 31);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
              const int r = wm0 + mi * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
              const float gq = __uint_as_float((uint32_t)f2bf(acc[mi][2 * pr][j]) << 16);
              const float uq = __uint_as_float((uint32_t)f2bf(acc[mi][2 * pr + 1][j]) << 16);
              cs[r * AP + fc] = f2bf(silu_f(gq) * uq);
            }
          }
        __syncthreads();
        constexpr int QPR = GBN / 16;  // 8-f chunks per row
        for (int u = tid; u < GBM * QPR; u += GNT) {
          const int r = u / QPR, q = u % QPR;
          const int f = nt * (GBN / 2) + q * 8;
          if (r >= mlen || f >= g.F) continue;
          *reinterpret_cast<u32x4*>(g.C + (int64_t)(mbase + r) * g.ldc + f) =
              *reinterpret_cast<const u32x4*>(&cs[r * AP + q * 8]);
        }
        return;
      }
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int r = wm0 + mi * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
          cs[r * CP + wn0 + ni * 32 + (lane & 31)] = f2bf(acc[mi][ni][j]);
        }
  }
  __syncthreads();
  const int BN = GBN, BM = GBM, NT = GNT;
  if constexpr (EPI == 1) {
    // tile column c: pair c/64, gate (c/32 even) or up (odd), f = nt*BN/2 + (c/64)*32 + c%32
    constexpr int UPR = BN / 16;  // gate chunks of 8 per row
    static_assert((BM * UPR) % NT == 0 && NT % 16 == 0, "every thread runs the same chunks of whole rows");
    if constexpr (F8) {
      if (g.aq != nullptr) {
        // act block-quantized for the down projection (the tile's 128 f are that product's k slice nt): the
        // four consecutive threads of one 32-f block (same row; q % 4 = 0..3) share its absmax, the block's
        // E8M0 exponent e is the smallest with absmax <= 448 * 2^e, and each element x * 2^-e (exact) is
        // rounded to e4m3; blocks past F get the scale byte of 1.0
        for (int u = tid; u < BM * UPR; u += NT) {
          const int r = u / UPR, q = u % UPR;
          const int cc = (q >> 2) * 64 + (q & 3) * 8;
          const int f = nt * (BN / 2) + (q >> 2) * 32 + (q & 3) * 8;
          const bool ok = r < mlen && f < g.F;
          const u32x4 gv = *reinterpret_cast<const u32x4*>(&cs[r * CP + cc]);
          const u32x4 uv = *reinterpret_cast<const u32x4*>(&cs[r * CP + cc + 32]);
          u32x4 av;
          float a[8];
          float amax = 0.f;
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const float g0 = __uint_as_float(gv[d] << 16), g1 = __uint_as_float(gv[d] & 0xffff0000u);
            const float u0 = __uint_as_float(uv[d] << 16), u1 = __uint_as_float(uv[d] & 0xffff0000u);
            av[d] = pack2bf(silu_f(g0) * u0, silu_f(g1) * u1);
            a[2 * d] = __uint_as_float(av[d] << 16);
            a[2 * d + 1] = __uint_as_float(av[d] & 0xffff0000u);
            amax = fmaxf(amax, fmaxf(fabsf(a[2 * d]), fabsf(a[2 * d + 1])));
          }
          amax = ok ? amax : 0.f;
          amax = fmaxf(amax, __shfl_xor(amax, 1));
          amax = fmaxf(amax, __shfl_xor(amax, 2));
          const int ex = mx_exponent(amax);
          const float sc = ldexpf(1.f, -ex);
          const int64_t row = mbase + r;
          if (ok) {
            int lo = 0, hi = 0;
            lo = __builtin_amdgcn_cvt_pk_fp8_f32(a[0] * sc, a[1] * sc, lo, false);
            lo = __builtin_amdgcn_cvt_pk_fp8_f32(a[2] * sc, a[3] * sc, lo, true);
            hi = __builtin_amdgcn_cvt_pk_fp8_f32(a[4] * sc, a[5] * sc, hi, false);
            hi = __builtin_amdgcn_cvt_pk_fp8_f32(a[6] * sc, a[7] * sc, hi, true);
            *reinterpret_cast<uint2*>(g.aq + row * g.F + f) = uint2{(unsigned)lo, (unsigned)hi};
            if (g.C != nullptr) *reinterpret_cast<u32x4*>(g.C + row * g.ldc + f) = av;
            if (g.C2 != nullptr) {
              *reinterpret_cast<u32x4*>(g.C2 + row * 2 * (int64_t)g.F + f) = gv;
              *reinterpret_cast<u32x4*>(g.C2 + row * 2 * (int64_t)g.F + g.F + f) = uv;
            }
          }
          if (r < mlen && (q & 3) == 0)
            g.aqs[((int64_t)nt * g.srows + row) * 4 + (q >> 2)] = (uint8_t)(f < g.F ? ex + 127 : 127);
        }
        return;
      }
    }
    for (int u = tid; u < BM * UPR; u += NT) {
      const int r = u / UPR, q = u % UPR;
      const int cc = (q >> 2) * 64 + (q & 3) * 8;  // gate column of this chunk
      const int f = nt * (BN / 2) + (q >> 2) * 32 + (q & 3) * 8;
      if (r >= mlen || f >= g.F) continue;
      const u32x4 gv = *reinterpret_cast<const u32x4*>(&cs[r * CP + cc]);
      const u32x4 uv = *reinterpret_cast<const u32x4*>(&cs[r * CP + cc + 32]);
      u32x4 av;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const float g0 = __uint_as_float(gv[d] << 16), g1 = __uint_as_float(gv[d] & 0xffff0000u);
        const float u0 = __uint_as_float(uv[d] << 16), u1 = __uint_as_float(uv[d] & 0xffff0000u);
        av[d] = pack2bf(silu_f(g0) * u0, silu_f(g1) * u1);
      }
      const int64_t row = mbase + r;
      *reinterpret_cast<u32x4*>(g.C + row * g.ldc + f) = av;
      if (g.C2 != nullptr) {  // the pre-activations, kept for the backward (none for inference)
        *reinterpret_cast<u32x4*>(g.C2 + row * 2 * (int64_t)g.F + f) = gv;
        *reinterpret_cast<u32x4*>(g.C2 + row * 2 * (int64_t)g.F + g.F + f) = uv;
      }
    }
  } else if constexpr (EPI == 2) {
    // SwiGLU backward: the pre-activations of 8 chunks per thread are requested together (clamped to the
    // tile's first row and column where a chunk lies outside the tile), so the HBM reads of the epilogue
    // overlap instead of costing one round trip per chunk
    constexpr int UPR = BN / 8;
    constexpr int PB = 8;
    static_assert((BM * UPR) % (NT * PB) == 0, "epilogue batches");
    for (int u0 = tid; u0 < BM * UPR; u0 += NT * PB) {
      u32x4 gvs[PB], uvs[PB];
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int u = u0 + i * NT;
        const int r = u / UPR, c = n0 + (u % UPR) * 8;
        const bool ok = r < mlen && c < g.N;
        const int64_t src = (int64_t)(mbase + (ok ? r : 0)) * 2 * g.F + (ok ? c : n0);
        gvs[i] = *reinterpret_cast<const u32x4*>(g.X + src);
        uvs[i] = *reinterpret_cast<const u32x4*>(g.X + src + g.F);
      }
#pragma unroll
      for (int i = 0; i < PB; ++i) {
        const int u = u0 + i * NT;
        const int r = u / UPR, cc = (u % UPR) * 8;
        const int c = n0 + cc;
        if (r >= mlen || c >= g.N) continue;
        const u32x4 v = *reinterpret_cast<const u32x4*>(&cs[r * CP + cc]);
        const int64_t row = mbase + r;
        const u32x4 gv = gvs[i], uv = uvs[i];
        u32x4 dg, du;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          float da[2] = {__uint_as_float(v[d] << 16), __uint_as_float(v[d] & 0xffff0000u)};
          float gg[2] = {__uint_as_float(gv[d] << 16), __uint_as_float(gv[d] & 0xffff0000u)};
          float uu[2] = {__uint_as_float(uv[d] << 16), __uint_as_float(uv[d] & 0xffff0000u)};
          float o1[2], o2[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float sg = sigmoid_f(gg[h]);
            const float sl = gg[h] * sg;
            o1[h] = da[h] * uu[h] * sg * (1.f + gg[h] * (1.f - sg));
            o2[h] = da[h] * sl;
          }
          dg[d] = pack2bf(o1[0], o1[1]);
          du[d] = pack2bf(o2[0], o2[1]);
        }
        *reinterpret_cast<u32x4*>(g.C + row * g.ldc + c) = dg;
        *reinterpret_cast<u32x4*>(g.C + row * g.ldc + g.F + c) = du;
      }
    }
  } else {
    constexpr int UPR = BN / 8;
    for (int u = tid; u < BM * UPR; u += NT) {
      const int r = u / UPR, cc = (u % UPR) * 8;
      const int c = n0 + cc;
      if (r >= mlen || c >= g.N) continue;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&cs[r * CP + cc]);
      if constexpr (GROUP == 0) {
        *reinterpret_cast<u32x4*>(g.C + (int64_t)(mbase + r) * g.ldc + c) = v;
      } else {
        const int m = mbase + r;
        const bool second = g.c_split > 0 && m >= g.c_split;
        uint16_t* base = (second ? g.C2 : g.C) + (int64_t)e * g.c_estride;
        *reinterpret_cast<u32x4*>(base + (int64_t)(second ? m - g.c_split : m) * g.ldc + c) = v;
      }
    }
  }
}

// tile_off[0] = 0, tile_off[e+1] = sum_{e' <= e} ceil(rows_e' / bm)  (one block, E <= 1024), and the
// expert order of the k-grouped products: experts ranked by rows (descending, lower id first on a tie) are
// dealt to the 8 XCD ranges in snake order (rank r -> range r % 8 on even rounds, 7 - r % 8 on odd ones),
// and korder lists range 0's experts by rank, then range 1's, ...
__global__ __launch_bounds__(1024) void k_gemm_tiles(const int* __restrict__ offsets, int E, int bm,
                                                     int* __restrict__ tile_off, int* __restrict__ korder) {
  __shared__ int part[1024];
  __shared__ int rows[1024];
  __shared__ int xcnt[8], xbase[8];
  const int tid = threadIdx.x;
  const int nrow = tid < E ? offsets[tid + 1] - offsets[tid] : 0;
  const int c = tid < E ? (nrow + bm - 1) / bm : 0;
  part[tid] = c;
  rows[tid] = nrow;
  if (tid < 8) xcnt[tid] = 0;
  __syncthreads();
  int rank = 0, x = 0, j = 0;
  if (tid < E) {
    for (int f = 0; f < E; ++f) rank += (rows[f] > nrow || (rows[f] == nrow && f < tid)) ? 1 : 0;
    j = rank >> 3;
    x = (j & 1) ? 7 - (rank & 7) : (rank & 7);
    atomicAdd(&xcnt[x], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int b = 0;
    for (int q = 0; q < 8; ++q) {
      xbase[q] = b;
      b += xcnt[q];
    }
  }
  __syncthreads();
  if (tid < E) korder[xbase[x] + j] = tid;
  for (int o = 1; o < 1024; o <<= 1) {
    const int v = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  if (tid == 0) tile_off[0] = 0;
  if (tid < E) tile_off[tid + 1] = part[tid];
}

namespace {
bool a16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
unsigned round8(int64_t v) { return (unsigned)((v + 7) / 8 * 8); }

template <int AM, int BMD, int GR, int EP, int NW>
int launch(const char* name, hipStream_t s, const GemmArgs& a, int64_t R) {
  int64_t blocks;
  if constexpr (GR == 0) {
    const int64_t Tn = EP == 1 ? (2 * (int64_t)a.F + GBN - 1) / GBN : ((int64_t)a.N + GBN - 1) / GBN;
    blocks = ((R + GBM - 1) / GBM + a.E) * Tn;
  } else {
    blocks = (int64_t)a.E * ((a.M + GBM - 1) / GBM) * ((a.N + GBN - 1) / GBN);
  }
  if (blocks <= 0) return 0;
  MOE_LAUNCH(name, (k_gemm<AM, BMD, GR, EP, NW>), dim3(round8(blocks)), dim3(NW * 64), 0, s, a);
  return check_launch(name);
}

constexpr int kTileBM = GBM;
// Wave layout per product: 4 waves of 128x128 (one per SIMD; register-staged refill two slices ahead) for the
// forward products (bf16 and fp8), whose operands are both k-contiguous; 8 waves of 128x64 (LDS-DMA refill)
// for the backward products.  The row-grouped tile prefix is computed with the kernels' BM.
constexpr int kNW_fwd1 = 4, kNW_fwd2 = 4, kNW_dact = 8, kNW_dxp = 8, kNW_dwd = 8, kNW_dw1 = 8, kNW_fp8 = 4;
}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_swiglu_workspace(int64_t E) { return (size_t)((2 * E + 1) * 4 + 255) & ~(size_t)255; }

extern "C" int moe_swiglu_fwd(const void* xp, const void* w_gate, const void* w_up, const void* w_down,
                              const int32_t* offsets, int64_t R, int64_t H, int64_t F, int64_t E, void* act,
                              void* hgu, void* y, void* workspace, size_t ws_bytes, void* stream) {
  if (R < 0 || H < 8 || F < 32 || E < 1 || E > 1024 || H % 8 || F % 32)
    return fail_arg("moe_swiglu_fwd: bad shape R=%lld H=%lld F=%lld E=%lld (need H%%8==0, F%%32==0)", (long long)R,
                    (long long)H, (long long)F, (long long)E);
  if (R == 0) return 0;
  if (!xp || !w_gate || !w_up || !w_down || !offsets || !act || !y || !a16(xp) || !a16(w_gate) ||
      !a16(w_up) || !a16(w_down) || !a16(act) || (hgu && !a16(hgu)) || !a16(y))
    return fail_arg("moe_swiglu_fwd: null or misaligned pointer");
  if (ws_bytes < moe_swiglu_workspace(E) || !workspace) return set_error("moe_swiglu_fwd: workspace"), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int* tile_off = static_cast<int*>(workspace);
  int* korder = tile_off + (E + 1);
  MOE_LAUNCH("k_gemm_tiles", k_gemm_tiles, dim3(1), dim3(1024), 0, s, offsets, (int)E, kTileBM, tile_off, korder);
  GemmArgs a{};
  a.offsets = offsets;
  a.tile_off = tile_off;
  a.E = (int)E;
  a.F = (int)F;
  // fwd1: [act | hgu] = xp . [Wg ; Wu]^T
  a.A = static_cast<const uint16_t*>(xp);
  a.lda = H;
  a.B = static_cast<const uint16_t*>(w_gate);
  a.B2 = static_cast<const uint16_t*>(w_up);
  a.ldb = H;
  a.b_estride = F * H;
  a.C = static_cast<uint16_t*>(act);
  a.C2 = static_cast<uint16_t*>(hgu);
  a.ldc = F;
  a.N = (int)(2 * F);
  a.K = (int)H;
  if (int rc = launch<0, 0, 0, 1, kNW_fwd1>("k_gemm_swiglu_fwd1", s, a, R)) return rc;
  // fwd2: y = act . Wd^T
  GemmArgs b{};
  b.offsets = offsets;
  b.tile_off = tile_off;
  b.E = (int)E;
  b.F = (int)F;
  b.A = static_cast<const uint16_t*>(act);
  b.lda = F;
  b.B = static_cast<const uint16_t*>(w_down);
  b.ldb = F;
  b.b_estride = H * F;
  b.C = static_cast<uint16_t*>(y);
  b.ldc = H;
  b.N = (int)H;
  b.K = (int)F;
  return launch<0, 0, 0, 0, kNW_fwd2>("k_gemm_swiglu_fwd2", s, b, R);
}

namespace moe {
namespace {
// fp8 forward workspace: tile prefix + expert order, then act in e4m3 [R, F], then its E8M0 block scales in the
// slice-major layout [(F / 128 slices) x srows rows x 4 blocks] (srows = R rounded up to 4) plus one 2 KB
// window of slack (the down projection stages 2 KB per slice from a tile's 4-aligned first row).
size_t fp8_act_bytes(int64_t R, int64_t F) { return ((size_t)R * F + 255) & ~(size_t)255; }
int64_t fp8_srows(int64_t R) { return (R + 3) / 4 * 4; }
size_t fp8_scale_bytes(int64_t R, int64_t F) {
  return (((size_t)((F + 127) / 128) * fp8_srows(R) * 4 + 2048) + 255) & ~(size_t)255;
}
}  // namespace
}  // namespace moe

extern "C" size_t moe_swiglu_fwd_fp8_workspace(int64_t R, int64_t F, int64_t E) {
  return moe_swiglu_workspace(E) + fp8_act_bytes(R, F) + fp8_scale_bytes(R, F);
}

extern "C" int moe_swiglu_fwd_fp8(const void* xq, const float* sx, const void* wg_q, const float* sg, const void* wu_q,
                                  const float* su, const void* wd_q, const float* sd, const int32_t* offsets, int64_t R,
                                  int64_t H, int64_t F, int64_t E, void* act, void* hgu, void* y, void* workspace,
                                  size_t ws_bytes, void* stream) {
  if (R < 0 || H < 16 || F < 32 || E < 1 || E > 1024 || H % 16 || F % 32)
    return fail_arg("moe_swiglu_fwd_fp8: bad shape R=%lld H=%lld F=%lld E=%lld (need H%%16==0, F%%32==0)",
                    (long long)R, (long long)H, (long long)F, (long long)E);
  if (R == 0) return 0;
  if (!xq || !sx || !wg_q || !sg || !wu_q || !su || !wd_q || !sd || !offsets || !y || !a16(xq) || !a16(wg_q) ||
      !a16(wu_q) || !a16(wd_q) || (act && !a16(act)) || (hgu && !a16(hgu)) || !a16(y))
    return fail_arg("moe_swiglu_fwd_fp8: null or misaligned pointer");
  if (ws_bytes < moe_swiglu_fwd_fp8_workspace(R, F, E) || !workspace)
    return set_error("moe_swiglu_fwd_fp8: workspace"), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int* tile_off = reinterpret_cast<int*>(ws);
  int* korder = tile_off + (E + 1);
  uint8_t* actq = reinterpret_cast<uint8_t*>(ws + moe_swiglu_workspace(E));
  uint8_t* sact = reinterpret_cast<uint8_t*>(ws + moe_swiglu_workspace(E) + fp8_act_bytes(R, F));
  MOE_LAUNCH("k_gemm_tiles", k_gemm_tiles, dim3(1), dim3(1024), 0, s, offsets, (int)E, kTileBM, tile_off, korder);
  // fwd1: [act | hgu] = (xq sx) . ([Wg ; Wu] [sg ; su])^T; fp8 matrices are addressed in 16-bit units
  GemmArgs a{};
  a.offsets = offsets;
  a.tile_off = tile_off;
  a.E = (int)E;
  a.F = (int)F;
  a.A = static_cast<const uint16_t*>(xq);
  a.lda = H / 2;
  a.B = static_cast<const uint16_t*>(wg_q);
  a.B2 = static_cast<const uint16_t*>(wu_q);
  a.ldb = H / 2;
  a.b_estride = F * H / 2;
  a.sa = sx;
  a.sb = sg;
  a.sb2 = su;
  a.C = static_cast<uint16_t*>(act);  // optional: act in bf16 as well
  a.C2 = static_cast<uint16_t*>(hgu);
  a.ldc = F;
  a.N = (int)(2 * F);
  a.K = (int)(H / 2);
  a.aq = actq;  // act block-quantized in the epilogue (e4m3 + E8M0 scale per 32 f)
  a.aqs = sact;
  a.srows = fp8_srows(R);
  if (int rc = launch<2, 2, 0, 1, kNW_fp8>("k_gemm_swiglu_fwd1_fp8", s, a, R)) return rc;
  // fwd2: y = (actq 2^e per block) . (Wd sd)^T, the block scales applied inside the MFMA
  GemmArgs b{};
  b.offsets = offsets;
  b.tile_off = tile_off;
  b.E = (int)E;
  b.F = (int)F;
  b.A = reinterpret_cast<const uint16_t*>(actq);
  b.lda = F / 2;
  b.B = static_cast<const uint16_t*>(wd_q);
  b.ldb = F / 2;
  b.b_estride = H * F / 2;
  b.mxs = sact;
  b.srows = fp8_srows(R);
  b.sb = sd;
  b.C = static_cast<uint16_t*>(y);
  b.ldc = H;
  b.N = (int)H;
  b.K = (int)(F / 2);
  return launch<2, 2, 0, 0, kNW_fp8>("k_gemm_swiglu_fwd2_fp8", s, b, R);
}

extern "C" int moe_swiglu_bwd(const void* dy, const void* xp, const void* act, const void* hgu, const void* w_gate,
                              const void* w_up, const void* w_down, const int32_t* offsets, int64_t R, int64_t H,
                              int64_t F, int64_t E, void* dh, void* dxp, void* dw_gate, void* dw_up, void* dw_down,
                              void* workspace, size_t ws_bytes, void* stream) {
  if (R < 0 || H < 8 || F < 32 || E < 1 || E > 1024 || H % 8 || F % 32)
    return fail_arg("moe_swiglu_bwd: bad shape R=%lld H=%lld F=%lld E=%lld (need H%%8==0, F%%32==0)", (long long)R,
                    (long long)H, (long long)F, (long long)E);
  if (!dy || !xp || !act || !hgu || !w_gate || !w_up || !w_down || !offsets || !dh || !dxp || !dw_gate || !dw_up ||
      !dw_down)
    return fail_arg("moe_swiglu_bwd: null pointer argument");
  if (ws_bytes < moe_swiglu_workspace(E) || !workspace) return set_error("moe_swiglu_bwd: workspace"), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int* tile_off = static_cast<int*>(workspace);
  int* korder = tile_off + (E + 1);
  MOE_LAUNCH("k_gemm_tiles", k_gemm_tiles, dim3(1), dim3(1024), 0, s, offsets, (int)E, kTileBM, tile_off, korder);
  // dA: dh = epilogue(dy . Wd)   (B[n=f][k=h] = Wd[h][f])
  if (R > 0) {
    GemmArgs a{};
    a.offsets = offsets;
    a.tile_off = tile_off;
    a.E = (int)E;
    a.F = (int)F;
    a.A = static_cast<const uint16_t*>(dy);
    a.lda = H;
    a.B = static_cast<const uint16_t*>(w_down);
    a.ldb = F;
    a.b_estride = H * F;
    a.C = static_cast<uint16_t*>(dh);
    a.ldc = 2 * F;
    a.X = static_cast<const uint16_t*>(hgu);
    a.N = (int)F;
    a.K = (int)H;
    if (int rc = launch<0, 1, 0, 2, kNW_dact>("k_gemm_swiglu_dact", s, a, R)) return rc;
  }
  // dxp = dh . [Wg ; Wu]   (B[n=h][k=j] = W1[j][h])
  if (R > 0) {
    GemmArgs a{};
    a.offsets = offsets;
    a.tile_off = tile_off;
    a.E = (int)E;
    a.F = (int)F;
    a.A = static_cast<const uint16_t*>(dh);
    a.lda = 2 * F;
    a.B = static_cast<const uint16_t*>(w_gate);
    a.B2 = static_cast<const uint16_t*>(w_up);
    a.b_split = (int)F;
    a.ldb = H;
    a.b_estride = F * H;
    a.C = static_cast<uint16_t*>(dxp);
    a.ldc = H;
    a.N = (int)H;
    a.K = (int)(2 * F);
    if (int rc = launch<0, 1, 0, 0, kNW_dxp>("k_gemm_swiglu_dxp", s, a, R)) return rc;
  }
  // dWd_e = dy_e^T . act_e   (M = H, N = F, K = rows of e)
  {
    GemmArgs a{};
    a.offsets = offsets;
    a.korder = korder;
    a.E = (int)E;
    a.A = static_cast<const uint16_t*>(dy);
    a.lda = H;
    a.B = static_cast<const uint16_t*>(act);
    a.ldb = F;
    a.C = static_cast<uint16_t*>(dw_down);
    a.ldc = F;
    a.c_estride = H * F;
    a.M = (int)H;
    a.N = (int)F;
    if (int rc = launch<1, 1, 1, 0, kNW_dwd>("k_gemm_swiglu_dwd", s, a, R)) return rc;
  }
  // [dWg_e ; dWu_e] = dh_e^T . xp_e   (M = 2F, N = H, K = rows of e)
  {
    GemmArgs a{};
    a.offsets = offsets;
    a.korder = korder;
    a.E = (int)E;
    a.A = static_cast<const uint16_t*>(dh);
    a.lda = 2 * F;
    a.B = static_cast<const uint16_t*>(xp);
    a.ldb = H;
    a.C = static_cast<uint16_t*>(dw_gate);
    a.C2 = static_cast<uint16_t*>(dw_up);
    a.c_split = (int)F;
    a.ldc = H;
    a.c_estride = F * H;
    a.M = (int)(2 * F);
    a.N = (int)H;
    return launch<1, 1, 1, 0, kNW_dw1>("k_gemm_swiglu_dw1", s, a, R);
  }
}

// ---------------------------------------------------------------------------
// MFMA ceiling (bench only): every CU runs one block of 8 waves (two per SIMD), each wave four independent
// accumulator chains of the GEMM's MFMA (bf16 v_mfma_f32_32x32x16_bf16, or the e4m3
// v_mfma_scale_f32_32x32x64_f8f6f4) with no memory traffic.  Wave 0 of each block stamps the shader clock
// counter (s_memtime) and the constant 100 MHz counter (s_memrealtime) around its loop, so the host gets
// the dense MFMA rate the chip sustains and the shader clock it runs at under that load.
// ---------------------------------------------------------------------------
namespace moe {
// Bits of random-looking operand data (a 32-bit integer hash of the lane, fragment and element).
__device__ __forceinline__ uint32_t ceil_hash(uint32_t v) {
  v ^= v >> 16;
  v *= 0x7feb352du;
  v ^= v >> 15;
  v *= 0x846ca68bu;
  v ^= v >> 16;
  return v;
}

// RAND: four independent A and four independent B fragments per lane, filled with hashed values (bf16: roughly
// uniform in [-2, 2); e4m3: any finite byte), re-paired on every MFMA of a statically unrolled group of four
// iterations, so consecutive MFMAs read different register data, as a data-carrying GEMM does; otherwise one A
// and one B fragment of near-constant values.
template <bool F8, bool RAND>
__global__ __launch_bounds__(512) void k_mfma_ceiling(int iters, unsigned long long* __restrict__ stamps,
                                                      float* __restrict__ sink) {
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  constexpr int NF = RAND ? 4 : 1;
  i32x8 fa[NF], fb[NF];
  bf16x8 ba[NF], bb[NF];
#pragma unroll
  for (int f = 0; f < NF; ++f)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if constexpr (RAND) {
        const uint32_t h = ceil_hash((threadIdx.x * 64u + (uint32_t)f * 8u + (uint32_t)i) * 2654435761u + blockIdx.x);
        const uint32_t h2 = ceil_hash(h ^ 0x9e3779b9u);
        fa[f][i] = (int)((h & 0x77777777u) | 0x08080808u);  // e4m3 bytes with exponent field < 15: finite
        fb[f][i] = (int)((h2 & 0x77777777u) | 0x08080808u);
        ba[f][i] = (__bf16)((float)(int)(h & 0xffffu) * (4.f / 65536.f) - 2.f);
        bb[f][i] = (__bf16)((float)(int)(h2 & 0xffffu) * (4.f / 65536.f) - 2.f);
      } else {
        fa[f][i] = 0x38383838 + (int)(threadIdx.x & 7);  // e4m3 bytes near 1.0
        fb[f][i] = 0x30303030 + i;
        ba[f][i] = (__bf16)(1e-3f * (float)(threadIdx.x + i));
        bb[f][i] = (__bf16)(2e-3f * (float)i);
      }
    }
  auto step = [&](int p) __attribute__((always_inline)) {
    // pairing p (0..NF-1): chain j multiplies A fragment (j + p) % NF by B fragment j
    if constexpr (F8) {
      c0 = mfma32x32x64_f8(fa[(0 + p) % NF], fb[0 % NF], c0);
      c1 = mfma32x32x64_f8(fa[(1 + p) % NF], fb[1 % NF], c1);
      c2 = mfma32x32x64_f8(fa[(2 + p) % NF], fb[2 % NF], c2);
      c3 = mfma32x32x64_f8(fa[(3 + p) % NF], fb[3 % NF], c3);
    } else {
      c0 = mfma32x32x16(ba[(0 + p) % NF], bb[0 % NF], c0);
      c1 = mfma32x32x16(ba[(1 + p) % NF], bb[1 % NF], c1);
      c2 = mfma32x32x16(ba[(2 + p) % NF], bb[2 % NF], c2);
      c3 = mfma32x32x16(ba[(3 + p) % NF], bb[3 % NF], c3);
    }
  };
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; it += NF) {
#pragma unroll
    for (int p = 0; p < NF; ++p) step(p);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  if (s == -1.2345e-30f) sink[0] = s;  // keeps the chains live; never true for these operands
  if (threadIdx.x == 0) {
    stamps[blockIdx.x * 2 + 0] = t1 - t0;
    stamps[blockIdx.x * 2 + 1] = r1 - r0;
  }
}
}  // namespace moe

// ---------------------------------------------------------------------------
// HBM ceiling probe (bench only): grid-stride streams of 16-byte accesses over buffers far larger than the
// caches, in the shapes the data-movement kernels have: read only, write only, copy, and fan-out (each
// 4 KB row read once and written to 6 rows, as the permute does at K = 6).  Streaming cache policy
// (non-temporal) throughout, as in those kernels.
// ---------------------------------------------------------------------------
namespace moe {
__global__ __launch_bounds__(256) void k_hbm_probe(int mode, const u32x4* __restrict__ x, u32x4* __restrict__ y,
                                                   int64_t n, unsigned* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (mode == 3) {  // fan-out: one wave per 4 KB row of x (n rows), written to rows r, r + n, ..., r + 5n of y
    const int lane = threadIdx.x & 63;
    for (int64_t r = t >> 6; r < n; r += stride >> 6) {
      u32x4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = __builtin_nontemporal_load(x + r * 256 + j * 64 + lane);
#pragma unroll
      for (int k = 0; k < 6; ++k)
#pragma unroll
        for (int j = 0; j < 4; ++j) __builtin_nontemporal_store(v[j], y + ((int64_t)k * n + r) * 256 + j * 64 + lane);
    }
    return;
  }
  unsigned acc = 0u;
  for (int64_t i = t; i < n; i += 4 * stride) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t k = i + u * stride;
      if (mode == 1) v[u] = u32x4{(unsigned)k, 1u, 2u, 3u};
      else v[u] = k < n ? __builtin_nontemporal_load(x + k) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t k = i + u * stride;
      if (mode == 0) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
      else if (k < n) __builtin_nontemporal_store(v[u], y + k);
    }
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // keeps the reads live
}
}  // namespace moe

extern "C" int moe_prof_hbm_ceiling(int64_t bytes, int mode, double* gbps) {
  if (bytes < (1 << 20) || bytes > ((int64_t)1 << 34) || mode < 0 || mode > 3 || !gbps)
    return fail_arg("moe_prof_hbm_ceiling: bad arguments (1 MiB <= bytes <= 16 GiB, mode 0..3, non-null output)");
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return check_launch("moe_prof_hbm_ceiling");
  // the buffer the mode moves `bytes` through: x read (modes 0, 2, 3), y written (modes 1, 2, 3)
  const int64_t rows = bytes / 4096;
  const int64_t xb = mode == 1 ? 16 : (mode == 3 ? rows * 4096 : bytes);
  const int64_t yb = mode == 0 ? 16 : (mode == 3 ? 6 * rows * 4096 : bytes);
  const int64_t n = mode == 3 ? rows : bytes / 16;
  const double moved = mode == 2 ? 2.0 * (double)bytes : (mode == 3 ? 7.0 * (double)rows * 4096 : (double)bytes);
  u32x4 *x = nullptr, *y = nullptr;
  unsigned* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  float ms = 0.f;
  if (hipMalloc(&x, (size_t)xb) != hipSuccess || hipMalloc(&y, (size_t)yb) != hipSuccess ||
      hipMalloc(&sink, 16) != hipSuccess || hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess ||
      hipMemsetAsync(x, 1, (size_t)xb, nullptr) != hipSuccess) {
    rc = check_launch("moe_prof_hbm_ceiling");
  } else {
    const int blocks = prop.multiProcessorCount * 8;
    auto run = [&]() { hipLaunchKernelGGL(k_hbm_probe, dim3(blocks), dim3(256), 0, nullptr, mode, x, y, n, sink); };
    for (int w = 0; w < 3; ++w) run();
    hipEventRecord(e0, nullptr);
    for (int r = 0; r < 10; ++r) run();
    hipEventRecord(e1, nullptr);
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
      rc = check_launch("moe_prof_hbm_ceiling");
  }
  if (rc == 0) *gbps = moved / ((double)ms / 10.0 * 1e-3) / 1e9;
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  if (x) hipFree(x);
  if (y) hipFree(y);
  if (sink) hipFree(sink);
  return rc;
}

extern "C" int moe_prof_mfma_ceiling(int64_t iters, int mode, double* tflops, double* clock_mhz) {
  if (iters < 1 || iters > (1 << 24) || mode < 0 || mode > 3 || !tflops || !clock_mhz)
    return fail_arg("moe_prof_mfma_ceiling: bad arguments (1 <= iters <= 2^24, mode 0..3, non-null outputs)");
  const bool fp8 = mode & 1, rnd = mode & 2;
  iters = (iters + 3) / 4 * 4;  // the random-operand loop runs groups of four iterations
  int dev = 0;
  hipDeviceProp_t prop;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return check_launch("moe_prof_mfma_ceiling");
  const int blocks = prop.multiProcessorCount;
  unsigned long long* d_st = nullptr;
  float* d_sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  int rc = 0;
  std::vector<unsigned long long> h((size_t)blocks * 2);
  float ms = 0.f;
  if (hipMalloc(&d_st, h.size() * sizeof(unsigned long long)) != hipSuccess || hipMalloc(&d_sink, 16) != hipSuccess ||
      hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    rc = check_launch("moe_prof_mfma_ceiling");
  } else {
    auto run = [&](int n) {
      if (fp8 && rnd)
        hipLaunchKernelGGL((k_mfma_ceiling<true, true>), dim3(blocks), dim3(512), 0, nullptr, n, d_st, d_sink);
      else if (fp8)
        hipLaunchKernelGGL((k_mfma_ceiling<true, false>), dim3(blocks), dim3(512), 0, nullptr, n, d_st, d_sink);
      else if (rnd)
        hipLaunchKernelGGL((k_mfma_ceiling<false, true>), dim3(blocks), dim3(512), 0, nullptr, n, d_st, d_sink);
      else
        hipLaunchKernelGGL((k_mfma_ceiling<false, false>), dim3(blocks), dim3(512), 0, nullptr, n, d_st, d_sink);
    };
    run((int)std::min<int64_t>(iters, 2000));  // warm the clocks
    hipEventRecord(e0, nullptr);
    run((int)iters);
    hipEventRecord(e1, nullptr);
    if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess ||
        hipMemcpy(h.data(), d_st, h.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost) != hipSuccess)
      rc = check_launch("moe_prof_mfma_ceiling");
  }
  if (rc == 0) {
    double sc = 0.0, sr = 0.0;
    for (int b = 0; b < blocks; ++b) {
      sc += (double)h[2 * b];
      sr += (double)h[2 * b + 1];
    }
    const double per_mfma = fp8 ? 2.0 * 32 * 32 * 64 : 2.0 * 32 * 32 * 16;
    *tflops = per_mfma * 4.0 * (double)iters * 8.0 * blocks / (ms * 1e-3) / 1e12;
    *clock_mhz = sr > 0.0 ? 100.0 * sc / sr : 0.0;
  }
  if (e0) hipEventDestroy(e0);
  if (e1) hipEventDestroy(e1);
  if (d_st) hipFree(d_st);
  if (d_sink) hipFree(d_sink);
  return rc;
}
