// DeBERTa-v2/v3 disentangled attention (forward), gfx950.
#include "attn_core.h"
#include "launch_util.h"

using namespace vfk;

extern "C" int vfk_flash_deberta_fwd(const vfk_tensor*, const vfk_tensor*, const vfk_tensor*,
                                     const int32_t*, const vfk_tensor*, const vfk_tensor*,
                                     int32_t, float, int32_t, int32_t, int32_t, vfk_tensor*,
                                     void*) {
  return set_error(VFK_ERR_UNSUPPORTED, "vfk_flash_deberta_fwd: not built yet");
}

extern "C" int vfk_deberta_fused_fwd(const vfk_tensor*, const vfk_tensor*, const vfk_tensor*,
                                     const int32_t*, const vfk_tensor*, const vfk_tensor*, float,
                                     int32_t, int32_t, int32_t, vfk_tensor*, void*) {
  return set_error(VFK_ERR_UNSUPPORTED, "vfk_deberta_fused_fwd: not built yet");
}
