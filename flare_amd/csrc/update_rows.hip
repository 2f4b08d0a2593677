// Update kernels instantiated for keyed sums (scatter, reduced gradients) in float32 or bfloat16 outputs.
#include "update.hpp"

namespace flare {

int launch_update_rows(int mode, const UpdateArgs &a, const Shape &sh, hipStream_t s) {
  if (mode == kModeRows) return launch_update_tag<TagF32, kModeRows>(a, sh, s);
  return launch_update_tag<TagF32, kModeUnique>(a, sh, s);
}

}  // namespace flare
