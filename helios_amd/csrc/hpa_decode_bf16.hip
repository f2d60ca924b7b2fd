// Decode kernels with bf16 queries and outputs (see hpa_decode_impl.h).
#include "hpa_decode_impl.h"

namespace hpa {
template DecodeFn pick_kv<BF16>(int, int, int, int);
}  // namespace hpa
