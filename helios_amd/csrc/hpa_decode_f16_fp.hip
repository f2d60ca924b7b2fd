// Decode kernels: f16 queries and outputs over f16 KV (hpa_decode_impl.h).
#include "hpa_decode_impl.h"

namespace hpa {
template DecodeFn pick_d<F16, F16, F32>(int, int);
}  // namespace hpa
