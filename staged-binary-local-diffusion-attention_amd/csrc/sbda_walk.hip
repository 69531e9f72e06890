// Wavefront-walk SBDA kernels (placeholder: not yet selected).
#include "sbda_params.h"

namespace sbda {

bool walk_applies(const Params&, int) { return false; }
hipError_t walk_forward(const Params&, int, bool, hipStream_t) { return hipErrorInvalidValue; }
hipError_t walk_backward(const Params&, int, bool, hipStream_t) { return hipErrorInvalidValue; }
void walk_partials(const Params&, int, int64_t* pq, int64_t* pk) { *pq = 0; *pk = 0; }

}  // namespace sbda
