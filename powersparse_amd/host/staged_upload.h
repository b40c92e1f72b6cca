// Host-to-device upload of large pageable arrays through page-locked staging.
#pragma once

#include <cstddef>

namespace PowerSparse {

// Copies `bytes` from host memory `src` (any, e.g. pageable) to device memory
// `dst` and returns when the copy is complete. Large copies go through two
// page-locked buffers: while the DMA engine copies chunk k out of one buffer,
// host threads fill the other with chunk k + 1. Small copies use one plain
// synchronous copy. Uses the current device's null stream.
void StagedUpload(void* dst, const void* src, size_t bytes);

}  // namespace PowerSparse
