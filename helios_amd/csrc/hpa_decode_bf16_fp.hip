// Decode kernels: bf16 queries and outputs over bf16 KV (hpa_decode_impl.h).
#include "hpa_decode_impl.h"

namespace hpa {
template DecodeFn pick_d<BF16, BF16, F32>(int, int);
}  // namespace hpa
