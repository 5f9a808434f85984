// Read-only HBM probe: the bandwidth ceiling a page-gathering reader can reach.
//
// The reference measures a bare copy_ as its practical ceiling (mini_vllm/bench.py:
// 448-466). On the MI355X a device copy moves read and write traffic at once and lands
// below what the paged decode itself reads, so it bounds nothing the decode does. This
// probe reads only, the way the decode does: whole pages of `page_bytes` (a paged pool's
// 16 rows x 8 kv heads x 128 bf16 = 32 KB), in the order a table gives (shuffled, as a
// pool is after many allocations) or in address order, each lane fetching 16-byte chunks
// with nontemporal loads, every load of a page in flight before any is used. The loaded
// words are folded into one value per lane and stored, so nothing is optimised away.
//
// One workgroup of 256 lanes per page at a time, pages taken in grid-stride order;
// `workgroups` sets how many are resident (the caller sweeps it).

#include "common.hpp"
#include "probe.hpp"

namespace mvllm {

namespace {

constexpr int kProbeThreads = 256;

template <int kChunks>  // 16-byte chunks per lane per page
__global__ __launch_bounds__(kProbeThreads) void read_pages_kernel(
    const char* __restrict__ base, const int32_t* __restrict__ pages, int64_t num_pages,
    int64_t page_bytes, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  for (int64_t i = blockIdx.x; i < num_pages; i += gridDim.x) {
    const int64_t page = pages != nullptr ? pages[i] : i;
    const u32x4* p = reinterpret_cast<const u32x4*>(base + page * page_bytes) + threadIdx.x;
    u32x4 v[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) v[c] = __builtin_nontemporal_load(p + c * kProbeThreads);
#pragma unroll
    for (int c = 0; c < kChunks; ++c) acc ^= v[c].x ^ v[c].y ^ v[c].z ^ v[c].w;
  }
  sink[static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x] = acc;
}

}  // namespace

bool read_probe_supported(int64_t page_bytes) {
  const int64_t per_lane = page_bytes / (16 * kProbeThreads);
  return page_bytes > 0 && page_bytes % (16 * kProbeThreads) == 0 &&
         (per_lane == 1 || per_lane == 2 || per_lane == 4 || per_lane == 8 || per_lane == 16);
}

int read_probe_sink_words(int32_t workgroups) { return workgroups * kProbeThreads; }

hipError_t launch_read_probe(const void* base, const int32_t* pages, int64_t num_pages,
                             int64_t page_bytes, int32_t workgroups, uint32_t* sink,
                             hipStream_t stream) {
  const char* b = static_cast<const char*>(base);
  switch (page_bytes / (16 * kProbeThreads)) {
    case 1: read_pages_kernel<1><<<workgroups, kProbeThreads, 0, stream>>>(b, pages, num_pages, page_bytes, sink); break;
    case 2: read_pages_kernel<2><<<workgroups, kProbeThreads, 0, stream>>>(b, pages, num_pages, page_bytes, sink); break;
    case 4: read_pages_kernel<4><<<workgroups, kProbeThreads, 0, stream>>>(b, pages, num_pages, page_bytes, sink); break;
    case 8: read_pages_kernel<8><<<workgroups, kProbeThreads, 0, stream>>>(b, pages, num_pages, page_bytes, sink); break;
    case 16: read_pages_kernel<16><<<workgroups, kProbeThreads, 0, stream>>>(b, pages, num_pages, page_bytes, sink); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace mvllm
