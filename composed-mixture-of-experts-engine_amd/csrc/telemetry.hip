// Per-step routing telemetry kept on the device.
//
// The reference's train step derives its routing telemetry from the router profile and the dispatch
// counts on the host, with .item() synchronisations every step (moe-engine/train.py L:360-399:
// expert_load_imbalance, router_z_loss, dead_expert_count, active_experts, routing_efficiency,
// dropped_token_fraction; RouterProfile fields from moe_router.py L:594-612, L:690-745).  Here one
// single-lane kernel turns the router's statistics vector (whose finalize already counts the experts
// without tokens) and the planner's drop count into one fixed-layout record of a ring buffer in device
// memory.  The ring's write cursor lives in device memory after the records and the kernel advances it
// with an atomic add, so a launch replayed from a HIP graph appends a new record each time; the caller
// copies the ring (cursor included) to the host only when it logs.
#include "common.h"

namespace moe {

// Record layout (floats).
enum TelField {
  kTelStep = 0,         // step number, stored as an int32 (the caller's, or the record's ordinal)
  kTelImbalance = 1,    // max(cnt) / mean(cnt)
  kTelZ = 2,            // mean_t logsumexp^2 (router_z_loss)
  kTelCntMean = 3,      // tokens_per_expert_mean
  kTelCntStd = 4,       // tokens_per_expert_std
  kTelDead = 5,         // dead_expert_count
  kTelActive = 6,       // active_experts
  kTelEfficiency = 7,   // routing_efficiency = dispatched / (capacity_factor * N * K)
  kTelDropped = 8,      // dropped_token_fraction = ndrop / (N * K)
  kTelAux = 9,          // aux statistic E * sum_e f_e P_e
  kTelNonfinite = 10,   // non-finite logits
  kTelDispatched = 11,  // dispatched slots (sum of cnt)
  kTelFields = 16       // record stride (16 floats = 64 bytes)
};

__global__ __launch_bounds__(64) void k_telemetry_record(const float* __restrict__ stats, int E, int64_t N, int K,
                                                         float capacity_factor, const int* __restrict__ ndrop,
                                                         int64_t step, float* __restrict__ ring, int capacity) {
  if (threadIdx.x != 0) return;
  int* cursor = reinterpret_cast<int*>(ring + (int64_t)capacity * kTelFields);
  const int n = atomicAdd(cursor, 1);  // records appended before this one
  float* rec = ring + (int64_t)(n % capacity) * kTelFields;
  const float dispatched = stats[5], dead = stats[7];
  const float cap = fmaxf(capacity_factor * (float)N * (float)K, 1.f);
  rec[kTelStep] = __int_as_float(step >= 0 ? (int)step : n);
  rec[kTelImbalance] = stats[2];
  rec[kTelZ] = stats[0];
  rec[kTelCntMean] = stats[3];
  rec[kTelCntStd] = stats[4];
  rec[kTelDead] = dead;
  rec[kTelActive] = (float)E - dead;
  rec[kTelEfficiency] = dispatched / cap;
  rec[kTelDropped] = (ndrop != nullptr && N > 0) ? (float)ndrop[0] / ((float)N * (float)K) : 0.f;
  rec[kTelAux] = stats[1];
  rec[kTelNonfinite] = stats[6];
  rec[kTelDispatched] = dispatched;
#pragma unroll
  for (int i = kTelDispatched + 1; i < kTelFields; ++i) rec[i] = 0.f;
}

}  // namespace moe

using namespace moe;

extern "C" int moe_telemetry_fields(void) { return kTelFields; }

extern "C" int moe_telemetry_record(const float* stats, int64_t E, int64_t N, int64_t K, float capacity_factor,
                                    const int32_t* ndrop, int64_t step, float* ring, int64_t capacity, void* stream) {
  if (E < 1 || N < 0 || K < 1 || step > INT32_MAX || capacity < 1 || capacity > (1 << 24))
    return fail_arg("moe_telemetry_record: bad arguments E=%lld N=%lld K=%lld step=%lld capacity=%lld",
                    (long long)E, (long long)N, (long long)K, (long long)step, (long long)capacity);
  if (!stats || !ring) return fail_arg("moe_telemetry_record: null pointer argument");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  MOE_LAUNCH("k_telemetry_record", k_telemetry_record, dim3(1), dim3(64), 0, s, stats, (int)E, N, (int)K,
             capacity_factor, ndrop, step, ring, (int)capacity);
  return check_launch("moe_telemetry_record");
}
