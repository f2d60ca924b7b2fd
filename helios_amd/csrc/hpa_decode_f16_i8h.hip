// Decode kernels: f16 queries and outputs over int8 KV with fp16 scales (hpa_decode_impl.h).
#include "hpa_decode_impl.h"

namespace hpa {
template DecodeFn pick_d<F16, I8, F16>(int, int);
}  // namespace hpa
