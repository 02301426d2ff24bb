// Compile-time constants (reference include/csrspmm/config.h:5).
#pragma once

namespace csrspmm {

// Lanes per wavefront on gfx950 (CDNA4 runs wave64); the reference's
// value is the 32-lane NVIDIA warp.
static constexpr int WARP_SIZE = 64;

}  // namespace csrspmm
