// _cumcount over arbitrary integer group ids (pkg/distributed/moe_layer.py L:64-115): for each element, the
// number of earlier elements (in input order) with the same id.
//
// The planner (dispatch.hip) computes the same quantity for ids that fit its key tables (at most 1024 distinct
// key values in one contiguous range).  This file covers every other input: the (id, position) pairs are sorted
// by id with rocPRIM's radix sort, which is stable -- equal ids keep their input order -- so an element's rank
// within its group is its sorted position minus the sorted position of its group's first element, found by a
// binary search over the sorted ids.  One kernel then writes each rank back to the element's input position.
// Integer work only, so the result is exact and independent of timing.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/iterator/counting_iterator.hpp>

#include "common.h"

namespace moe {
namespace {

// out[pos[i]] = i - (first sorted index whose id equals key[i]).
__global__ __launch_bounds__(256) void k_cumcount_rank(const int64_t* __restrict__ key, const int* __restrict__ pos,
                                                       int64_t n, int64_t* __restrict__ out) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    const int64_t k = key[i];
    int64_t lo = 0, hi = i;  // first index in [0, i] with key == k (the keys are sorted ascending)
    while (lo < hi) {
      const int64_t mid = (lo + hi) >> 1;
      if (key[mid] < k) lo = mid + 1;
      else hi = mid;
    }
    out[pos[i]] = i - lo;
  }
}

size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

struct CumWs {
  size_t off_keys, off_pos, off_tmp, tmp_bytes, total;
};

CumWs cum_ws(int64_t n) {
  CumWs w{};
  size_t tmp = 0;
  rocprim::counting_iterator<int> iota(0);
  (void)rocprim::radix_sort_pairs(nullptr, tmp, static_cast<const int64_t*>(nullptr), static_cast<int64_t*>(nullptr),
                                  iota, static_cast<int*>(nullptr), (size_t)n);
  w.off_keys = 0;
  w.off_pos = al256((size_t)n * 8);
  w.off_tmp = w.off_pos + al256((size_t)n * 4);
  w.tmp_bytes = tmp;
  w.total = w.off_tmp + al256(tmp);
  return w;
}

}  // namespace
}  // namespace moe

using namespace moe;

extern "C" size_t moe_cumcount_workspace(int64_t n) {
  if (n <= 0 || n > INT32_MAX) return 0;
  return cum_ws(n).total;
}

extern "C" int moe_cumcount(const int64_t* groups, int64_t n, int64_t* out, void* workspace, size_t ws_bytes,
                            void* stream) {
  if (n < 0 || n > INT32_MAX) return fail_arg("moe_cumcount: n=%lld out of range", (long long)n);
  if (n == 0) return 0;
  if (!groups || !out) return fail_arg("moe_cumcount: null pointer argument");
  const CumWs w = cum_ws(n);
  if (!workspace || ws_bytes < w.total)
    return set_error("moe_cumcount: workspace %zu < %zu bytes", ws_bytes, w.total), MOE_EWORKSPACE;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  int64_t* keys = reinterpret_cast<int64_t*>(ws + w.off_keys);
  int* pos = reinterpret_cast<int*>(ws + w.off_pos);
  size_t tmp = w.tmp_bytes;
  rocprim::counting_iterator<int> iota(0);
  hipError_t e = rocprim::radix_sort_pairs(ws + w.off_tmp, tmp, groups, keys, iota, pos, (size_t)n, 0u, 64u, s);
  if (e != hipSuccess) return set_error("moe_cumcount: radix sort: %s", hipGetErrorString(e)), (int)e;
  MOE_LAUNCH("k_cumcount_rank", k_cumcount_rank, dim3((unsigned)std::min<int64_t>(4096, (n + 255) / 256)),
             dim3(256), 0, s, keys, pos, n, out);
  return check_launch("moe_cumcount");
}
