// MI355X shape constants, shared by device code and by host-only builds (no HIP headers).
#pragma once

namespace mla {

constexpr int kWave = 64;      // CDNA wavefront width
constexpr int kNumCUs = 256;   // MI355X: 8 XCDs x 32 CUs
constexpr int kNumXCDs = 8;

}  // namespace mla
