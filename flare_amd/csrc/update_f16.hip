// Update kernels instantiated for optimizer updates of float16 tables.
#include "update.hpp"

namespace flare {

int launch_update_f16(int mode, const UpdateArgs &a, const Shape &sh, hipStream_t s) {
  if (mode == kModeSgd) return launch_update_tag<TagF16, kModeSgd>(a, sh, s);
  if (mode == kModeAdam) return launch_update_tag<TagF16, kModeAdam>(a, sh, s);
  return launch_update_tag<TagF16, kModeAdagrad>(a, sh, s);
}

}  // namespace flare
