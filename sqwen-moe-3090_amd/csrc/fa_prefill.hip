// fa_prefill.hip - MFMA FlashAttention for prefill chunks (n_q * H/Hkv > 16).
#include "common.hpp"

namespace sqa {

size_t fa_prefill_workspace(int64_t, int64_t, int64_t) { return 0; }

int launch_fa_prefill(const FaArgs &, hipStream_t) {
    return set_error(SQA_ERR_UNSUPPORTED, "flash_attn_ext: prefill kernel not built");
}

}  // namespace sqa
