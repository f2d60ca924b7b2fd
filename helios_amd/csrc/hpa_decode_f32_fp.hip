// Decode kernels: f32 queries and outputs over f32 KV (hpa_decode_impl.h).
#include "hpa_decode_impl.h"

namespace hpa {
template DecodeFn pick_d<F32, F32, F32>(int, int);
}  // namespace hpa
