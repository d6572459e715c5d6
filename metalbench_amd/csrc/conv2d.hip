// placeholder translation unit; the conv2d kernel lands here next.
#include "common.h"
namespace mb {
void register_conv2d() {}
}  // namespace mb
extern "C" int mb_launch_conv2d_nhwc_f32(const float*, const float*, float*, uint32_t, uint32_t,
                                         uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                                         uint32_t, uint32_t, void*) {
    return mb::fail(MB_E_NOT_FOUND, "conv2d_nhwc_f32 not built yet");
}
