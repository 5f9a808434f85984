// Internal interface of the read-only HBM probe (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvllm {

// Pages of page_bytes: a multiple of 4 KB, 4-64 KB.
bool read_probe_supported(int64_t page_bytes);
// uint32 words the sink must hold for `workgroups`.
int read_probe_sink_words(int32_t workgroups);
// Reads num_pages pages of page_bytes from base (page i at pages[i], or i when pages is
// null) and stores one folded word per lane in sink.
hipError_t launch_read_probe(const void* base, const int32_t* pages, int64_t num_pages,
                             int64_t page_bytes, int32_t workgroups, uint32_t* sink,
                             hipStream_t stream);

}  // namespace mvllm
