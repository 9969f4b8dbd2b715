// prefill.hip — MFMA flash-attention prefill (placeholder until the kernel lands).
#include "vva_internal.hpp"

namespace vva {

bool prefill_supported(const AttnArgs&) { return false; }
hipError_t launch_prefill(const AttnArgs&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace vva
