// Decode kernels with f16 queries and outputs (see hpa_decode_impl.h).
#include "hpa_decode_impl.h"

namespace hpa {
template DecodeFn pick_kv<F16>(int, int, int, int);
}  // namespace hpa
