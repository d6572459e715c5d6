// placeholder translation unit; the decoder step lands here next.
#include "common.h"
namespace mb {
void register_decoder() {}
}  // namespace mb
extern "C" uint64_t mb_decoder_step_workspace_bytes(const mb_decoder_step_args*) {
    mb::fail(MB_E_NOT_FOUND, "decoder step not built yet");
    return 0;
}
extern "C" int mb_launch_llama_decoder_step_bf16(const mb_decoder_step_args*, void*) {
    return mb::fail(MB_E_NOT_FOUND, "decoder step not built yet");
}
