// Router statistics finalize shared by the router kernels: per-block partials (dispatch counts,
// probability sums, z sums, non-finite counts) written through to the coherence point, and the fixed-order
// fold of all of them into cnt / stats / aux / z by one block (stats[7]: experts that received no token).
#pragma once

#include "common.h"

namespace moe {

constexpr int kMaxK = 32;
constexpr int kMaxE = 256;

// Per-block partials handed to the last block of the same launch.  They are stored and loaded as
// agent-scope relaxed atomics: the stores write through the XCD-local L2 to the coherence point and the
// loads bypass it, so no L2 writeback / invalidate (buffer_wbl2 / buffer_inv) is needed around the ticket
// -- those flush every dirty line of the L2, including data earlier kernels left there.
template <typename T>
__device__ __forceinline__ void st_part(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool COH, typename T>
__device__ __forceinline__ T ld_part(const T* p) {
  if constexpr (COH) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else return *p;
}

// ---------------------------------------------------------------------------
// Finalize: fixed-order sums of the per-block partials -> cnt, stats, aux, z (one block of NTHR threads).
// ---------------------------------------------------------------------------
// LDS scratch the finalize needs (floats).
template <int NTHR>
constexpr int finalize_scratch_floats() { return 2 * kMaxE + 2 * (NTHR / 64) + 8 * NTHR; }

template <int NTHR, bool COH = false>
__device__ __forceinline__ void router_finalize_block(const int* __restrict__ part_cnt, const float* __restrict__ part_p,
                                                      const float* __restrict__ part_z, int nblk, int N, int E, int K,
                                                      float aux_coef, float z_coef, int64_t* __restrict__ cnt_out,
                                                      float* __restrict__ stats, float* __restrict__ aux_out,
                                                      float* __restrict__ z_out, float* scratch) {
  float* s_c = scratch;                                                       // [kMaxE]
  float* s_pe = scratch + kMaxE;                                              // [kMaxE]
  float(*s_red)[NTHR / 64] = reinterpret_cast<float(*)[NTHR / 64]>(scratch + 2 * kMaxE);  // [2][NTHR/64]
  int* s_pc = reinterpret_cast<int*>(scratch + 2 * kMaxE + 2 * (NTHR / 64));  // [nj][E] <= 4 * NTHR
  float* s_pp = scratch + 2 * kMaxE + 2 * (NTHR / 64) + 4 * NTHR;             // [nj][E]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Per-expert sums over the blocks.  Thread (jj, q) = (tid / nq, tid % nq) owns V consecutive experts
  // (V = 4 when E % 4 == 0: one 16-byte load per array and block) and sums blocks jj, jj + nj, ... (experts
  // fastest across lanes, so a load instruction reads consecutive experts of one block); a pairwise tree over
  // jj in LDS then folds the nj partial sums (a fixed order for a given block count).
  {
    const bool quad = (E & 3) == 0;
    const int V = quad ? 4 : 1;
    const int nq = E / V;
    // nj block strides: a power of two, at most NTHR / nq, and about nblk / 8 so each thread sums
    // several blocks (loads in flight) and the tree fold below stays short
    int nj = 1;
    while (2 * nj * nq <= NTHR && 2 * nj <= (nblk + 7) / 8) nj *= 2;
    const int q = tid % nq;
    const int jj = tid / nq;
    int c[4] = {0, 0, 0, 0};
    float p[4] = {0.f, 0.f, 0.f, 0.f};
    if (jj < nj) {
      if (quad) {
        const buf_rsrc_t rc = buf_rsrc(part_cnt, nblk * E * 4), rp = buf_rsrc(part_p, nblk * E * 4);
        constexpr int pol = COH ? kPolicyCoherent : 0;
        int b = jj;
        for (; b + 7 * nj < nblk; b += 8 * nj) {  // 16 independent 16-byte loads in flight
          u32x4 cv[8], pv[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int off = ((b + u * nj) * E + 4 * q) * 4;
            cv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, pol));
            pv[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, pol));
          }
#pragma unroll
          for (int u = 0; u < 8; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              c[i] += (int)cv[u][i];
              p[i] += __uint_as_float(pv[u][i]);
            }
        }
        for (; b < nblk; b += nj) {
          const int off = (b * E + 4 * q) * 4;
          const u32x4 cv = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, pol));
          const u32x4 pv = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, off, 0, pol));
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            c[i] += (int)cv[i];
            p[i] += __uint_as_float(pv[i]);
          }
        }
      } else {
        int b = jj;
        for (; b + 7 * nj < nblk; b += 8 * nj) {  // 8 independent loads in flight
          int cv[8];
          float pv[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            cv[u] = ld_part<COH>(&part_cnt[(int64_t)(b + u * nj) * E + q]);
            pv[u] = ld_part<COH>(&part_p[(int64_t)(b + u * nj) * E + q]);
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            c[0] += cv[u];
            p[0] += pv[u];
          }
        }
        for (; b < nblk; b += nj) {
          c[0] += ld_part<COH>(&part_cnt[(int64_t)b * E + q]);
          p[0] += ld_part<COH>(&part_p[(int64_t)b * E + q]);
        }
      }
    }
    // partial sums land in LDS at [jj][expert]
    if (jj < nj) {
      for (int i = 0; i < V; ++i) {
        s_pc[jj * E + q * V + i] = c[i];
        s_pp[jj * E + q * V + i] = p[i];
      }
    }
    __syncthreads();
    // pairwise tree over jj (fixed order): row j += row j + half
    for (int half = nj >> 1; half > 0; half >>= 1) {
      for (int i = tid; i < half * E; i += NTHR) {
        s_pc[i] += s_pc[i + half * E];
        s_pp[i] += s_pp[i + half * E];
      }
      __syncthreads();
    }
    if (tid < E) {
      const int cs = s_pc[tid];
      const float ps = s_pp[tid];
      cnt_out[tid] = cs;
      s_c[tid] = (float)cs;
      s_pe[tid] = ps / (float)N;
      stats[MOE_STATS_HEAD + tid] = ps / (float)N;
    }
  }
  float z = 0.f, nf = 0.f;
  {
    int b = tid;
    for (; b + 3 * NTHR < nblk; b += 4 * NTHR) {
      f32x4 zz;
      float nn[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        zz[u] = ld_part<COH>(&part_z[2 * (b + u * NTHR)]);
        nn[u] = ld_part<COH>(&part_z[2 * (b + u * NTHR) + 1]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        z += zz[u];
        nf += nn[u];
      }
    }
    for (; b < nblk; b += NTHR) {
      z += ld_part<COH>(&part_z[2 * b]);
      nf += ld_part<COH>(&part_z[2 * b + 1]);
    }
  }
  z = wave_sum(z);
  nf = wave_sum(nf);
  if (lane == 0) {
    s_red[0][tid >> 6] = z;
    s_red[1][tid >> 6] = nf;
  }
  __syncthreads();
  if (tid < 64) {  // wave 0: the per-expert statistics in double, lane-strided then a fixed butterfly
    double tot = 0.0, mx = 0.0, aux = 0.0;
    int dead = 0;
    for (int e = tid; e < E; e += 64) {
      const double c = s_c[e];
      tot += c;
      mx = fmax(mx, c);
      aux += (c / ((double)N * K)) * (double)s_pe[e];
      dead += c == 0.0;
    }
    tot = wave_sum(tot);
    aux = wave_sum(aux);
    dead = wave_sum(dead);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
    const double mean = tot / E;
    double var = 0.0;
    for (int e = tid; e < E; e += 64) var += ((double)s_c[e] - mean) * ((double)s_c[e] - mean);
    var = wave_sum(var);
    if (tid != 0) return;
    z = s_red[0][0];
    nf = s_red[1][0];
    for (int w = 1; w < NTHR / 64; ++w) {
      z += s_red[0][w];
      nf += s_red[1][w];
    }
    const float zstat = z / (float)N;
    const float aux_raw = (float)(aux * E);
    stats[0] = zstat;
    stats[1] = aux_raw;
    stats[2] = mean < 1e-9 ? 1.f : (float)(mx / mean);
    stats[3] = (float)mean;
    stats[4] = E > 1 ? (float)sqrt(var / (E - 1)) : NAN;
    stats[5] = (float)tot;
    stats[6] = nf;
    stats[7] = (float)dead;
    if (aux_out) aux_out[0] = aux_coef * aux_raw;
    if (z_out) z_out[0] = z_coef * zstat;
  }
}

// ---------------------------------------------------------------------------
// Router backward without dx, for callers that form dx from G themselves (the norm-fused backward):
// dwg = x^T G reduced over token chunks into dwg_out (bf16 [H, E]), and G = dL/dlogits rounded to bf16
// written to g_out ([N, g_pitch], experts past E zero; g_pitch = 8 or 16).  Applies to bf16 x and gate
// with E <= 16 and H % 256 == 0; ws holds router_dw_g_workspace(N, H, E) bytes.
// ---------------------------------------------------------------------------
bool router_dw_g_applies(int64_t H, int64_t E);
size_t router_dw_g_workspace(int64_t N, int64_t H, int64_t E);
int router_dw_g(const uint16_t* x, const uint16_t* wg, const float* logits, const int64_t* idx, const void* grad_w,
                int gw_dtype, const int64_t* cnt, const float* grad_aux, const float* grad_z, float aux_coef,
                float z_coef, int64_t N, int64_t H, int64_t E, int64_t K, void* dwg_out, uint16_t* g_out, int g_pitch,
                void* ws, hipStream_t s);

}  // namespace moe
