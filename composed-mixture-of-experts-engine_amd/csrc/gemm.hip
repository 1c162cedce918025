// Grouped SwiGLU expert GEMMs for gfx950 (bf16 in, fp32 accumulate).
//
// One kernel template covers the six products of the expert FFN forward and
// backward.  Each computes C[m, n] = sum_k A[m, k] B[n, k] on
// v_mfma_f32_32x32x16_bf16 with 128x128x64 block tiles, 4 waves of 64x64, a
// double-buffered LDS pipeline (k-contiguous rows, 16-byte fragment reads)
// and a register stage for the next k-tile's global loads.
//
//   operand mode 0 ("rows"): element (i, k) at P[i*ld + k]  (k contiguous,
//                            copied to LDS with 16-byte stores)
//   operand mode 1 ("cols"): element (i, k) at P[k*ld + i]  (i contiguous,
//                            transposed into LDS with 2-byte stores)
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
//
// products (R = rows, per expert e):
//   fwd1  [act | hgu] = xp  . [Wg_e ; Wu_e]^T      A rows(xp), B rows(W),  G0, EPI1
//   fwd2  y           = act . Wd_e^T               A rows,     B rows,     G0, EPI0
//   dA    dh          = dy  . Wd_e  (+ epilogue)   A rows,     B cols(Wd), G0, EPI2
//   dxp   dxp         = dh  . [Wg_e ; Wu_e]        A rows,     B cols(W),  G0, EPI0
//   dWd   dWd_e       = dy_e^T . act_e             A cols,     B cols,     G1, EPI0
//   dW1   [dWg_e;dWu_e] = dh_e^T . xp_e            A cols,     B cols,     G1, EPI0
#include <algorithm>

#include "common.h"

namespace moe {

struct GemmArgs {
  const uint16_t* A;   // A operand source
  int64_t lda;
  const uint16_t* B;   // B operand source (first half when b_split > 0)
  const uint16_t* B2;  // second B source: used for B index >= b_split (k for cols, n for EPI1)
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
  const int* tile_off; // [E+1] tile prefix (row-grouped)
  int E;
  int M, N, K;         // k-grouped: M, N fixed; row-grouped: N, K fixed
  int mtiles;          // k-grouped: tiles along M
};

constexpr int GBM = 128, GBN = 128, GBK = 64, GPITCH = GBK + 8;

__device__ __forceinline__ float silu_f(float g) { return g / (1.f + __expf(-g)); }

template <int AMODE, int BMODE, int GROUP, int EPI>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t As[2][GBM * GPITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][GBN * GPITCH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int wm = wv >> 1;
  const int wn = wv & 1;

  // ---- tile decode ----
  int e, mbase, mlen, kbase, klen;
  const int n0 = blockIdx.y * GBN;
  if constexpr (GROUP == 0) {
    const int tile = blockIdx.x;
    const int total = g.tile_off[g.E];
    if (tile >= total) return;
    int lo = 0, hi = g.E - 1;  // largest e with tile_off[e] <= tile
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (g.tile_off[mid] <= tile) lo = mid;
      else hi = mid - 1;
    }
    e = lo;
    const int seg0 = g.offsets[e];
    mbase = seg0 + (tile - g.tile_off[e]) * GBM;
    mlen = min(GBM, g.offsets[e + 1] - mbase);
    kbase = 0;
    klen = g.K;
  } else {
    e = blockIdx.x / g.mtiles;
    mbase = (blockIdx.x % g.mtiles) * GBM;
    mlen = min(GBM, g.M - mbase);
    kbase = g.offsets[e];
    klen = g.offsets[e + 1] - kbase;
  }
  const int nlen = (EPI == 1) ? min(GBN, 2 * (g.F - blockIdx.y * (GBN / 2))) : min(GBN, g.N - n0);

  // ---- global -> register staging ----
  u32x4 ra[4], rb[4];
  const u32x4 zero4 = u32x4{0u, 0u, 0u, 0u};

  auto b_row_ptr = [&](int c, int k) -> const uint16_t* {
    // B element (tile column c, absolute k) for BMODE 0 (rows)
    if constexpr (EPI == 1) {
      const int f = blockIdx.y * (GBN / 2) + (c >> 6) * 32 + (c & 31);
      const uint16_t* base = ((c >> 5) & 1) ? g.B2 : g.B;
      return base + (int64_t)e * g.b_estride + (int64_t)f * g.ldb + k;
    } else {
      return g.B + (int64_t)e * g.b_estride + (int64_t)(n0 + c) * g.ldb + k;
    }
  };

  auto load_tile = [&](int k0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = tid + 256 * j;
      if constexpr (AMODE == 0) {
        const int r = q >> 3, kc = q & 7;
        const int k = k0 + kc * 8;
        const bool ok = r < mlen && k < klen;
        ra[j] = ok ? *reinterpret_cast<const u32x4*>(g.A + (int64_t)(mbase + r) * g.lda + kbase + k) : zero4;
      } else {
        const int kk = q >> 4, mc = q & 15;
        const int m = mbase + mc * 8;
        const bool ok = (k0 + kk) < klen && m < g.M;
        ra[j] = ok ? *reinterpret_cast<const u32x4*>(g.A + (int64_t)(kbase + k0 + kk) * g.lda + m) : zero4;
      }
      if constexpr (BMODE == 0) {
        const int c = q >> 3, kc = q & 7;
        const int k = k0 + kc * 8;
        const bool ok = c < nlen && k < klen;
        rb[j] = ok ? *reinterpret_cast<const u32x4*>(b_row_ptr(c, kbase + k)) : zero4;
      } else {
        const int kk = q >> 4, nc = q & 15;
        const int n = n0 + nc * 8;
        const int k = k0 + kk;
        const bool ok = k < klen && n < g.N;
        if (ok) {
          const uint16_t* p;
          if constexpr (GROUP == 0) {
            const bool second = g.b_split > 0 && k >= g.b_split;
            const int kr = second ? k - g.b_split : k;
            p = (second ? g.B2 : g.B) + (int64_t)e * g.b_estride + (int64_t)kr * g.ldb + n;
          } else {
            p = g.B + (int64_t)(kbase + k) * g.ldb + n;
          }
          rb[j] = *reinterpret_cast<const u32x4*>(p);
        } else {
          rb[j] = zero4;
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
    uint16_t* as = As[buf];
    uint16_t* bs = Bs[buf];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = tid + 256 * j;
      if constexpr (AMODE == 0) {
        *reinterpret_cast<u32x4*>(&as[(q >> 3) * GPITCH + (q & 7) * 8]) = ra[j];
      } else {
        const int kk = q >> 4, mc = q & 15;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          as[(mc * 8 + 2 * i) * GPITCH + kk] = (uint16_t)(ra[j][i] & 0xffffu);
          as[(mc * 8 + 2 * i + 1) * GPITCH + kk] = (uint16_t)(ra[j][i] >> 16);
        }
      }
      if constexpr (BMODE == 0) {
        *reinterpret_cast<u32x4*>(&bs[(q >> 3) * GPITCH + (q & 7) * 8]) = rb[j];
      } else {
        const int kk = q >> 4, nc = q & 15;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bs[(nc * 8 + 2 * i) * GPITCH + kk] = (uint16_t)(rb[j][i] & 0xffffu);
          bs[(nc * 8 + 2 * i + 1) * GPITCH + kk] = (uint16_t)(rb[j][i] >> 16);
        }
      }
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[mi][ni][j] = 0.f;

  const int nk = (klen + GBK - 1) / GBK;
  if (nk > 0) {
    load_tile(0);
    store_tile(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      if (kt + 1 < nk) load_tile((kt + 1) * GBK);
      const uint16_t* as = As[buf];
      const uint16_t* bs = Bs[buf];
#pragma unroll
      for (int ks = 0; ks < GBK / 16; ++ks) {
        i16x8 fa[2], fb[2];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
          fa[mi] = *reinterpret_cast<const i16x8*>(
              &as[(wm * 64 + mi * 32 + (lane & 31)) * GPITCH + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
          fb[ni] = *reinterpret_cast<const i16x8*>(
              &bs[(wn * 64 + ni * 32 + (lane & 31)) * GPITCH + ks * 16 + (lane >> 5) * 8]);
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
          for (int ni = 0; ni < 2; ++ni)
            acc[mi][ni] = mfma32x32x16(__builtin_bit_cast(bf16x8, fa[mi]), __builtin_bit_cast(bf16x8, fb[ni]),
                                       acc[mi][ni]);
      }
      if (kt + 1 < nk) store_tile(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: acc[mi][ni][j] = C[wm*64 + mi*32 + (j/4)*8 + (lane/32)*4 + j%4][wn*64 + ni*32 + lane%32] ----
#pragma unroll
  for (int mi = 0; mi < 2; ++mi) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int r = wm * 64 + mi * 32 + (j >> 2) * 8 + (lane >> 5) * 4 + (j & 3);
      if (r >= mlen) continue;
      if constexpr (EPI == 1) {
        const int f = blockIdx.y * (GBN / 2) + wn * 32 + (lane & 31);
        if (f < g.F) {
          const float gv = acc[mi][0][j];
          const float uv = acc[mi][1][j];
          const int64_t row = mbase + r;
          g.C[row * g.ldc + f] = f2bf(silu_f(gv) * uv);
          g.C2[row * 2 * (int64_t)g.F + f] = f2bf(gv);
          g.C2[row * 2 * (int64_t)g.F + g.F + f] = f2bf(uv);
        }
      } else {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
          const int c = n0 + wn * 64 + ni * 32 + (lane & 31);
          if (c >= g.N) continue;
          const float v = acc[mi][ni][j];
          if constexpr (EPI == 2) {
            const int64_t row = mbase + r;
            const float gv = bf2f(g.X[row * 2 * (int64_t)g.F + c]);
            const float uv = bf2f(g.X[row * 2 * (int64_t)g.F + g.F + c]);
            const float sg = 1.f / (1.f + __expf(-gv));
            const float sl = gv * sg;
            const float dsl = sg * (1.f + gv * (1.f - sg));
            g.C[row * g.ldc + c] = f2bf(v * uv * dsl);
            g.C[row * g.ldc + g.F + c] = f2bf(v * sl);
          } else if constexpr (GROUP == 0) {
            g.C[(int64_t)(mbase + r) * g.ldc + c] = f2bf(v);
          } else {
            const int m = mbase + r;
            const bool second = g.c_split > 0 && m >= g.c_split;
            uint16_t* base = (second ? g.C2 : g.C) + (int64_t)e * g.c_estride;
            base[(int64_t)(second ? m - g.c_split : m) * g.ldc + c] = f2bf(v);
          }
        }
      }
    }
  }
}

// tile_off[0] = 0, tile_off[e+1] = sum_{e' <= e} ceil(rows_e' / GBM)  (one block, E <= 1024).
__global__ __launch_bounds__(1024) void k_gemm_tiles(const int* __restrict__ offsets, int E, int* __restrict__ tile_off) {
  __shared__ int part[1024];
  const int tid = threadIdx.x;
  const int c = tid < E ? (offsets[tid + 1] - offsets[tid] + GBM - 1) / GBM : 0;
  part[tid] = c;
  __syncthreads();
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

template <int AM, int BM_, int GR, int EP>
int launch(const char* name, dim3 grid, hipStream_t s, const GemmArgs& a) {
  MOE_LAUNCH(name, (k_gemm<AM, BM_, GR, EP>), grid, dim3(256), 0, s, a);
  return check_launch(name);
}
}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_swiglu_workspace(int64_t E) { return (size_t)((E + 1) * 4 + 255) & ~(size_t)255; }

extern "C" int moe_swiglu_fwd(const void* xp, const void* w_gate, const void* w_up, const void* w_down,
                              const int32_t* offsets, int64_t R, int64_t H, int64_t F, int64_t E, void* act,
                              void* hgu, void* y, void* workspace, size_t ws_bytes, void* stream) {
  if (R < 0 || H < 8 || F < 32 || E < 1 || E > 1024 || H % 8 || F % 32)
    return fail_arg("moe_swiglu_fwd: bad shape R=%lld H=%lld F=%lld E=%lld (need H%%8==0, F%%32==0)", (long long)R,
                    (long long)H, (long long)F, (long long)E);
  if (R == 0) return 0;
  if (!xp || !w_gate || !w_up || !w_down || !offsets || !act || !hgu || !y || !a16(xp) || !a16(w_gate) ||
      !a16(w_up) || !a16(w_down) || !a16(act) || !a16(hgu) || !a16(y))
    return fail_arg("moe_swiglu_fwd: null or misaligned pointer");
  if (ws_bytes < moe_swiglu_workspace(E) || !workspace) return set_error("moe_swiglu_fwd: workspace"), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  int* tile_off = static_cast<int*>(workspace);
  MOE_LAUNCH("k_gemm_tiles", k_gemm_tiles, dim3(1), dim3(1024), 0, s, offsets, (int)E, tile_off);
  const unsigned mt = (unsigned)((R + GBM - 1) / GBM + E);
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
  if (int rc = launch<0, 0, 0, 1>("k_gemm_swiglu_fwd1", dim3(mt, (unsigned)((F + 63) / 64)), s, a)) return rc;
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
  return launch<0, 0, 0, 0>("k_gemm_swiglu_fwd2", dim3(mt, (unsigned)((H + GBN - 1) / GBN)), s, b);
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
  MOE_LAUNCH("k_gemm_tiles", k_gemm_tiles, dim3(1), dim3(1024), 0, s, offsets, (int)E, tile_off);
  const unsigned mt = (unsigned)((std::max<int64_t>(R, 1) + GBM - 1) / GBM + E);
  // dA: dh = epilogue(dy . Wd)   (B[n=f][k=h] = Wd[h][f])
  {
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
    if (R > 0)
      if (int rc = launch<0, 1, 0, 2>("k_gemm_swiglu_dact", dim3(mt, (unsigned)((F + GBN - 1) / GBN)), s, a)) return rc;
  }
  // dxp = dh . [Wg ; Wu]   (B[n=h][k=j] = W1[j][h])
  {
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
    if (R > 0)
      if (int rc = launch<0, 1, 0, 0>("k_gemm_swiglu_dxp", dim3(mt, (unsigned)((H + GBN - 1) / GBN)), s, a)) return rc;
  }
  // dWd_e = dy_e^T . act_e   (M = H, N = F, K = rows of e)
  {
    GemmArgs a{};
    a.offsets = offsets;
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
    a.mtiles = (int)((H + GBM - 1) / GBM);
    if (int rc = launch<1, 1, 1, 0>("k_gemm_swiglu_dwd", dim3((unsigned)(E * a.mtiles), (unsigned)((F + GBN - 1) / GBN)),
                                    s, a))
      return rc;
  }
  // [dWg_e ; dWu_e] = dh_e^T . xp_e   (M = 2F, N = H, K = rows of e)
  {
    GemmArgs a{};
    a.offsets = offsets;
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
    a.mtiles = (int)((2 * F + GBM - 1) / GBM);
    return launch<1, 1, 1, 0>("k_gemm_swiglu_dw1", dim3((unsigned)(E * a.mtiles), (unsigned)((H + GBN - 1) / GBN)),
                              s, a);
  }
}
