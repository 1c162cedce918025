// Grouped SwiGLU expert GEMMs in float32 (the reference module's default dtype) for gfx950.
//
// The same six products as the bf16 kernels (gemm.hip) -- C[m, n] = sum_k A[m, k] B[n, k] per expert segment,
// with the SwiGLU forward / backward fused into the epilogues -- on v_mfma_f32_32x32x2_f32: float32 products and
// float32 sums, as the reference's float32 F.linear computes them (pkg/distributed/moe_layer.py L:166-198,
// L:326-337).  The fp32 MFMA peak is 1/16 of the bf16 one, so each block is small enough that two share a CU:
// 128x128 tiles, four waves of 64x64 (2 x 2 MFMA blocks of 32 x 32), 16-wide k slices double-buffered in LDS and
// refilled through registers one slice ahead.
//
// LDS holds each operand tile as [i][k] (k contiguous, row pitch 20 floats): a lane reads four consecutive k of
// its row with one 16-byte read and feeds them to four MFMAs.  An MFMA may take its two k values from any
// positions as long as A and B agree: in MFMA s of a group of 8 k, lane l supplies k = 8 grp + 4 (l / 32) + s for
// its row (A) or column (B), so the four MFMAs of a group cover its 8 k once each.
//   operand mode 0 ("rows"): element (i, k) at P[i*ld + k]: 16-byte global loads along k, copied to LDS as is
//   operand mode 1 ("cols"): element (i, k) at P[k*ld + i]: 16-byte global loads along i, written to LDS
//                            transposed (four 4-byte writes)
//   GROUP 0: rows of one expert segment (tile prefix from k_gemm_tiles with bm = 128); GROUP 1: the reduction
//   runs over the expert's rows (weight gradients; experts without rows get zeros).
//   EPI 0 store C; EPI 1 SwiGLU forward (the B tile interleaves 32 gate and 32 up rows, so a lane holds g and u
//   of the same (row, f) in its two n blocks): act = silu(g) u and hgu = [g | u]; EPI 2 SwiGLU backward from
//   C = dA and hgu: dh = [dA u silu'(g) | dA silu(g)].
#include "common.h"

namespace moe {

struct GemmF32Args {
  const float* A;
  int64_t lda;
  const float* B;
  const float* B2;     // second B source: k >= b_split (cols mode) / up rows (EPI 1)
  int64_t ldb;
  int64_t b_estride;   // per-expert stride of B / B2 (row-grouped)
  int b_split;
  float* C;
  float* C2;           // EPI 1: hgu; k-grouped: rows >= c_split
  int64_t ldc;
  int64_t c_estride;   // per-expert stride of C / C2 (k-grouped)
  int c_split;
  const float* X;      // EPI 2: hgu
  int F;
  const int* offsets;  // [E+1]
  const int* tile_off; // [E+1] m-tile prefix with bm = 128 (row-grouped)
  int E;
  int M, N, K;         // k-grouped: M, N; row-grouped: N, K
};

constexpr int FBM = 128, FBN = 128, FBK = 16;
constexpr int FKP = FBK + 4;  // LDS row pitch (floats): 80 bytes, keeps 16-byte reads aligned

__device__ __forceinline__ f32x16 mfma32x32x2_f32(float a, float b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// silu and its derivative in float32 with the library exponential (the reference's torch silu, x / (1 + e^-x))
__device__ __forceinline__ float sig32(float g) { return 1.f / (1.f + expf(-g)); }

template <int AMODE, int BMODE, int GROUP, int EPI>
__global__ __launch_bounds__(256, 2) void k_gemm_f32(GemmF32Args g) {
  __shared__ __attribute__((aligned(16))) float sa[2][FBM * FKP];
  __shared__ __attribute__((aligned(16))) float sb[2][FBN * FKP];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int wm0 = (wv >> 1) * 64, wn0 = (wv & 1) * 64;

  // ---- tile decode (the grid is sized for the most tiles any routing can produce; surplus blocks exit) ----
  int e, mbase, mlen, kbase, klen, nt;
  if constexpr (GROUP == 0) {
    const int Tn = (EPI == 1) ? (2 * g.F + FBN - 1) / FBN : (g.N + FBN - 1) / FBN;
    const int L = (int)blockIdx.x;
    if (L >= g.tile_off[g.E] * Tn) return;
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
    mbase = g.offsets[e] + mt * FBM;
    mlen = min(FBM, g.offsets[e + 1] - mbase);
    kbase = 0;
    klen = g.K;
  } else {
    const int Tm = (g.M + FBM - 1) / FBM, Tn = (g.N + FBN - 1) / FBN;
    const int L = (int)blockIdx.x;
    if (L >= g.E * Tm * Tn) return;
    e = L / (Tm * Tn);
    const int r = L - e * Tm * Tn;
    const int mt = r / Tn;
    nt = r - mt * Tn;
    mbase = mt * FBM;
    mlen = min(FBM, g.M - mbase);
    kbase = g.offsets[e];
    klen = g.offsets[e + 1] - kbase;
  }
  const int n0 = nt * FBN;
  const int nlen = (EPI == 1) ? min(FBN, 2 * (g.F - nt * (FBN / 2))) : min(FBN, g.N - n0);
  const int nk = (klen + FBK - 1) / FBK;

  // ---- operand sources.  Rows mode: thread q = tid + 256 j loads row q / 4, k chunk (q % 4) * 4 of the slice;
  // cols mode: k-row q / 32, i chunk (q % 32) * 4.  Rows / columns past the tile are clamped to valid ones
  // (their results are never stored); k past the reduction reads zeros. ----
  const float* arow[2];
  const float* brow[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int q = tid + 256 * j;
    if constexpr (AMODE == 0) {
      const int i = min(q >> 2, mlen - 1);
      arow[j] = g.A + (int64_t)(mbase + i) * g.lda + kbase + (q & 3) * 4;
    } else {
      const int ic = (q & 31) * 4;
      arow[j] = g.A + (int64_t)kbase * g.lda + mbase + (ic < mlen ? ic : 0);
    }
    if constexpr (BMODE == 0) {
      const int i = min(q >> 2, nlen - 1);
      if constexpr (EPI == 1) {
        const int f = nt * (FBN / 2) + (i >> 6) * 32 + (i & 31);
        brow[j] = (((i >> 5) & 1) ? g.B2 : g.B) + (int64_t)e * g.b_estride + (int64_t)f * g.ldb + (q & 3) * 4;
      } else {
        brow[j] = g.B + (int64_t)e * g.b_estride + (int64_t)(n0 + i) * g.ldb + (q & 3) * 4;
      }
    } else {
      const int ic = (q & 31) * 4;
      const int off = n0 + (ic < nlen ? ic : 0);
      if constexpr (GROUP == 0) brow[j] = g.B + (int64_t)e * g.b_estride + off;
      else brow[j] = g.B + (int64_t)kbase * g.ldb + off;
    }
  }
  const float* b2row0 = nullptr;  // cols-mode B with a split (dxp): the second source's column base
  if constexpr (BMODE == 1 && GROUP == 0) {
    const int ic = (tid & 31) * 4;
    b2row0 = g.b_split > 0 ? g.B2 + (int64_t)e * g.b_estride + n0 + (ic < nlen ? ic : 0) : nullptr;
  }

  f32x4 ra[2], rb[2];
  auto load = [&](int kt) {
    const int k0 = kt * FBK;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = tid + 256 * j;
      if constexpr (AMODE == 0) {
        const int k = k0 + (q & 3) * 4;
        ra[j] = k < klen ? *reinterpret_cast<const f32x4*>(arow[j] + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        const int k = k0 + (q >> 5);
        ra[j] = k < klen ? *reinterpret_cast<const f32x4*>(arow[j] + (int64_t)k * g.lda) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
      if constexpr (BMODE == 0) {
        const int k = k0 + (q & 3) * 4;
        rb[j] = k < klen ? *reinterpret_cast<const f32x4*>(brow[j] + k0) : f32x4{0.f, 0.f, 0.f, 0.f};
      } else {
        const int k = k0 + (q >> 5);
        const float* src;
        if constexpr (GROUP == 0) {
          // both j of a thread share its column (256 is a multiple of 32), so the second source's column base
          // b2row0 serves both
          if (g.b_split > 0 && k >= g.b_split) src = b2row0 + (int64_t)(k - g.b_split) * g.ldb;
          else src = brow[j] + (int64_t)k * g.ldb;
        } else {
          src = brow[j] + (int64_t)k * g.ldb;
        }
        rb[j] = k < klen ? *reinterpret_cast<const f32x4*>(src) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = tid + 256 * j;
      if constexpr (AMODE == 0) {
        *reinterpret_cast<f32x4*>(&sa[buf][(q >> 2) * FKP + (q & 3) * 4]) = ra[j];
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) sa[buf][((q & 31) * 4 + d) * FKP + (q >> 5)] = ra[j][d];
      }
      if constexpr (BMODE == 0) {
        *reinterpret_cast<f32x4*>(&sb[buf][(q >> 2) * FKP + (q & 3) * 4]) = rb[j];
      } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) sb[buf][((q & 31) * 4 + d) * FKP + (q >> 5)] = rb[j][d];
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mi][ni][r] = 0.f;

  if (nk > 0) {
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      if (kt + 1 < nk) load(kt + 1);  // in flight during this slice's MFMAs
#pragma unroll
      for (int grp = 0; grp < 2; ++grp) {
        f32x4 fa[2], fb[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
          fa[mi] = *reinterpret_cast<const f32x4*>(
              &sa[buf][(wm0 + mi * 32 + (lane & 31)) * FKP + grp * 8 + (lane >> 5) * 4]);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          fb[ni] = *reinterpret_cast<const f32x4*>(
              &sb[buf][(wn0 + ni * 32 + (lane & 31)) * FKP + grp * 8 + (lane >> 5) * 4]);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
          for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32x32x2_f32(fa[mi][s], fb[ni][s], acc[mi][ni]);
      }
      if (kt + 1 < nk) {
        store(buf ^ 1);  // the other buffer was last read in slice kt-1, before the barrier that ended it
        __syncthreads();
      }
    }
  }

  // ---- epilogue straight from the accumulators: acc[mi][ni][r] = C[wm0 + mi*32 + 8 (r/4) + 4 (lane/32) + r%4]
  // [wn0 + ni*32 + lane%32]; 32 lanes of a row write 128 consecutive bytes ----
  const int jl = lane & 31;
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ri = wm0 + mi * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (ri >= mlen) continue;
      const int64_t row = mbase + ri;
      if constexpr (EPI == 1) {
        // the wave's two n blocks: gate (ni = 0) and up (ni = 1) of the same 32 f
        const int f = nt * (FBN / 2) + (wn0 >> 6) * 32 + jl;
        if (f >= g.F) continue;
        const float gv = acc[mi][0][r], uv = acc[mi][1][r];
        g.C[row * g.ldc + f] = gv * sig32(gv) * uv;
        if (g.C2 != nullptr) {
          g.C2[row * 2 * (int64_t)g.F + f] = gv;
          g.C2[row * 2 * (int64_t)g.F + g.F + f] = uv;
        }
      } else {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          const int c = n0 + wn0 + ni * 32 + jl;
          if (c >= g.N) continue;
          const float v = acc[mi][ni][r];
          if constexpr (EPI == 2) {
            const float gv = g.X[row * 2 * (int64_t)g.F + c], uv = g.X[row * 2 * (int64_t)g.F + g.F + c];
            const float sg = sig32(gv);
            g.C[row * g.ldc + c] = v * uv * sg * (1.f + gv * (1.f - sg));
            g.C[row * g.ldc + g.F + c] = v * gv * sg;
          } else if constexpr (GROUP == 0) {
            g.C[row * g.ldc + c] = v;
          } else {
            const bool second = g.c_split > 0 && row >= g.c_split;
            float* base = (second ? g.C2 : g.C) + (int64_t)e * g.c_estride;
            base[(second ? row - g.c_split : row) * g.ldc + c] = v;
          }
        }
      }
    }
}

__global__ void k_gemm_tiles_f32(const int* __restrict__ offsets, int E, int* __restrict__ tile_off) {
  // tile_off[e+1] = sum_{e' <= e} ceil(rows_e' / 128), one thread (E <= 1024: a few microseconds)
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    int acc = 0;
    tile_off[0] = 0;
    for (int e = 0; e < E; ++e) {
      acc += (offsets[e + 1] - offsets[e] + FBM - 1) / FBM;
      tile_off[e + 1] = acc;
    }
  }
}

namespace {
bool a16f(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <int AM, int BMD, int GR, int EP>
int launch_f32(const char* name, hipStream_t s, const GemmF32Args& a, int64_t R) {
  int64_t blocks;
  if constexpr (GR == 0) {
    const int64_t Tn = EP == 1 ? (2 * (int64_t)a.F + FBN - 1) / FBN : ((int64_t)a.N + FBN - 1) / FBN;
    blocks = ((R + FBM - 1) / FBM + a.E) * Tn;
  } else {
    blocks = (int64_t)a.E * ((a.M + FBM - 1) / FBM) * ((a.N + FBN - 1) / FBN);
  }
  if (blocks <= 0) return 0;
  MOE_LAUNCH(name, (k_gemm_f32<AM, BMD, GR, EP>), dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_launch(name);
}

int check_f32(const char* what, int64_t R, int64_t H, int64_t F, int64_t E) {
  if (R < 0 || H < 4 || F < 32 || E < 1 || E > 1024 || H % 4 || F % 32)
    return fail_arg("%s: bad shape R=%lld H=%lld F=%lld E=%lld (need H%%4==0, F%%32==0, E<=1024)", what,
                    (long long)R, (long long)H, (long long)F, (long long)E);
  return 0;
}
}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_swiglu_f32_workspace(int64_t E) { return (size_t)((E + 1) * 4 + 255) & ~(size_t)255; }

extern "C" int moe_swiglu_fwd_f32(const float* xp, const float* w_gate, const float* w_up, const float* w_down,
                                  const int32_t* offsets, int64_t R, int64_t H, int64_t F, int64_t E, float* act,
                                  float* hgu, float* y, void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = check_f32("moe_swiglu_fwd_f32", R, H, F, E)) return rc;
  if (R == 0) return 0;
  if (!xp || !w_gate || !w_up || !w_down || !offsets || !act || !y || !a16f(xp) || !a16f(w_gate) || !a16f(w_up) ||
      !a16f(w_down))
    return fail_arg("moe_swiglu_fwd_f32: null or misaligned pointer");
  if (!workspace || ws_bytes < moe_swiglu_f32_workspace(E))
    return set_error("moe_swiglu_fwd_f32: workspace"), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int* tile_off = static_cast<int*>(workspace);
  MOE_LAUNCH("k_gemm_tiles_f32", k_gemm_tiles_f32, dim3(1), dim3(64), 0, s, offsets, (int)E, tile_off);
  GemmF32Args a{};
  a.offsets = offsets;
  a.tile_off = tile_off;
  a.E = (int)E;
  a.F = (int)F;
  // fwd1: [act | hgu] = xp . [Wg ; Wu]^T
  a.A = xp;
  a.lda = H;
  a.B = w_gate;
  a.B2 = w_up;
  a.ldb = H;
  a.b_estride = F * H;
  a.C = act;
  a.C2 = hgu;
  a.ldc = F;
  a.N = (int)(2 * F);
  a.K = (int)H;
  if (int rc = launch_f32<0, 0, 0, 1>("k_gemm_swiglu_fwd1_f32", s, a, R)) return rc;
  // fwd2: y = act . Wd^T
  GemmF32Args b{};
  b.offsets = offsets;
  b.tile_off = tile_off;
  b.E = (int)E;
  b.F = (int)F;
  b.A = act;
  b.lda = F;
  b.B = w_down;
  b.ldb = F;
  b.b_estride = H * F;
  b.C = y;
  b.ldc = H;
  b.N = (int)H;
  b.K = (int)F;
  return launch_f32<0, 0, 0, 0>("k_gemm_swiglu_fwd2_f32", s, b, R);
}

extern "C" int moe_swiglu_bwd_f32(const float* dy, const float* xp, const float* act, const float* hgu,
                                  const float* w_gate, const float* w_up, const float* w_down, const int32_t* offsets,
                                  int64_t R, int64_t H, int64_t F, int64_t E, float* dh, float* dxp, float* dw_gate,
                                  float* dw_up, float* dw_down, void* workspace, size_t ws_bytes, void* stream) {
  if (int rc = check_f32("moe_swiglu_bwd_f32", R, H, F, E)) return rc;
  if (!dy || !xp || !act || !hgu || !w_gate || !w_up || !w_down || !offsets || !dh || !dxp || !dw_gate || !dw_up ||
      !dw_down)
    return fail_arg("moe_swiglu_bwd_f32: null pointer argument");
  if (!a16f(dy) || !a16f(xp) || !a16f(act) || !a16f(dh) || !a16f(w_gate) || !a16f(w_up) || !a16f(w_down))
    return fail_arg("moe_swiglu_bwd_f32: operands must be 16-byte aligned");
  if (!workspace || ws_bytes < moe_swiglu_f32_workspace(E))
    return set_error("moe_swiglu_bwd_f32: workspace"), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int* tile_off = static_cast<int*>(workspace);
  MOE_LAUNCH("k_gemm_tiles_f32", k_gemm_tiles_f32, dim3(1), dim3(64), 0, s, offsets, (int)E, tile_off);
  if (R > 0) {
    // dA: dh = epilogue(dy . Wd)   (B[n = f][k = h] = Wd[h][f])
    GemmF32Args a{};
    a.offsets = offsets;
    a.tile_off = tile_off;
    a.E = (int)E;
    a.F = (int)F;
    a.A = dy;
    a.lda = H;
    a.B = w_down;
    a.ldb = F;
    a.b_estride = H * F;
    a.C = dh;
    a.ldc = 2 * F;
    a.X = hgu;
    a.N = (int)F;
    a.K = (int)H;
    if (int rc = launch_f32<0, 1, 0, 2>("k_gemm_swiglu_dact_f32", s, a, R)) return rc;
    // dxp = dh . [Wg ; Wu]   (B[n = h][k = j] = W1[j][h])
    GemmF32Args b{};
    b.offsets = offsets;
    b.tile_off = tile_off;
    b.E = (int)E;
    b.F = (int)F;
    b.A = dh;
    b.lda = 2 * F;
    b.B = w_gate;
    b.B2 = w_up;
    b.b_split = (int)F;
    b.ldb = H;
    b.b_estride = F * H;
    b.C = dxp;
    b.ldc = H;
    b.N = (int)H;
    b.K = (int)(2 * F);
    if (int rc = launch_f32<0, 1, 0, 0>("k_gemm_swiglu_dxp_f32", s, b, R)) return rc;
  }
  // dWd_e = dy_e^T . act_e   (M = H, N = F, K = rows of e)
  GemmF32Args c{};
  c.offsets = offsets;
  c.E = (int)E;
  c.A = dy;
  c.lda = H;
  c.B = act;
  c.ldb = F;
  c.C = dw_down;
  c.ldc = F;
  c.c_estride = H * F;
  c.M = (int)H;
  c.N = (int)F;
  if (int rc = launch_f32<1, 1, 1, 0>("k_gemm_swiglu_dwd_f32", s, c, R)) return rc;
  // [dWg_e ; dWu_e] = dh_e^T . xp_e   (M = 2F, N = H, K = rows of e)
  GemmF32Args d{};
  d.offsets = offsets;
  d.E = (int)E;
  d.A = dh;
  d.lda = 2 * F;
  d.B = xp;
  d.ldb = H;
  d.C = dw_gate;
  d.C2 = dw_up;
  d.c_split = (int)F;
  d.ldc = H;
  d.c_estride = F * H;
  d.M = (int)(2 * F);
  d.N = (int)H;
  return launch_f32<1, 1, 1, 0>("k_gemm_swiglu_dw1_f32", s, d, R);
}
