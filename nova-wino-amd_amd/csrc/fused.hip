// Fused transform + MFMA + transform kernel (placeholder: not yet enabled).
#include "nova_internal.h"

namespace nova {

bool fused_supported(int K, int C) {
    (void)K;
    (void)C;
    return false;
}

hipError_t launch_fused(const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int,
                        int, int, int, int, int, int, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace nova
