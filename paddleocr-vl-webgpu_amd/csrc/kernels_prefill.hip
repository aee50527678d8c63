// Causal prefill (placeholder until the MFMA kernel lands).
#include <hip/hip_runtime.h>

#include "pvlc_internal.hpp"

namespace pvlc {

int launch_prefill(const pvlc_hip_paged_prefill_args *, void *) { return static_cast<int>(hipErrorNotSupported); }

}  // namespace pvlc
