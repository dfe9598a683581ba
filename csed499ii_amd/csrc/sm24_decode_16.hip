// Decode-kernel launchers for 16-column tiles (grouped and per-column scales): one
// translation unit per tile width, so that the library compiles in parallel.
#include "sm24_decode_launch.h"

namespace sm24 {
SM24_DECODE_INSTANTIATE(16)
}  // namespace sm24
