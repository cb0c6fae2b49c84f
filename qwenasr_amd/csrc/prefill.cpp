// decoder_prefill (decoder.rs:455-547) on the device.
#include "decoder.h"

void decoder_free_prefill(qasr_decoder *d) {
    PrefillBufs &p = d->pf;
    for (float *b : {p.x, p.xn, p.qkv, p.att, p.gu, p.g})
        if (b) (void)hipFree(b);
    p = PrefillBufs{};
}

extern "C" int qasr_hip_decoder_prefill(qasr_decoder *d, const float *embeds, int64_t seq_len) {
    if (!d) return qasr_fail(QASR_ERR_INVALID, "decoder is null");
    (void)embeds;
    (void)seq_len;
    return qasr_fail(QASR_ERR_INVALID, "decoder_prefill: not available in this build");
}
