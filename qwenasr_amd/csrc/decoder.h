// Internal layout of the device-resident decoder.
#pragma once
#include <array>
#include <map>
#include <vector>
#include "kernels.h"
#include "model.h"

struct DecLayerDev {
    // int8 packed (decode) and bf16 (prefill) weights, row-major [out, in]
    int8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wdown = nullptr;
    float *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sdown = nullptr;
    uint16_t *bqkv = nullptr, *bo = nullptr, *bgu = nullptr, *bdown = nullptr;
    float *q_norm = nullptr, *k_norm = nullptr, *in_norm = nullptr, *post_norm = nullptr;
};

struct PrefillBufs {
    int64_t cap = 0;
    float *x = nullptr, *xn = nullptr, *qkv = nullptr, *att = nullptr, *gu = nullptr, *g = nullptr;
};

struct qasr_decoder {
    qasr_hip *h = nullptr;
    qasr_dec_config c{};
    int round_mode = 0, kv_bf16 = 0;
    int64_t max_seq = 0, len = 0;
    std::vector<DecLayerDev> L;
    uint16_t *embed = nullptr;
    int8_t *lm = nullptr;                       // int8 decode head [lm_i8_rows][hidden] + row scales
    float *lm_s = nullptr, *norm = nullptr;
    int64_t lm_i8_rows = 0;                     // cfg.lm_head_dim(): vocab, or the aligner's classify_num
    uint16_t *lm_bf16 = nullptr;                // separate bf16 LM head for prefill logits (nullptr: tied embedding)
    int64_t lm_rows = 0;
    void *kc = nullptr, *vc = nullptr;          // [layer][kv_head][max_seq][hd]
    int64_t kv_layer_stride = 0;                // prefill's cache elements between layers (0: kv_heads * max_seq * hd)
    float *rc = nullptr, *rs = nullptr;         // RoPE [max_seq][hd]
    float *rope_cur = nullptr;                  // [2][hd]: cos, sin rows of the step's position
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *ffn = nullptr;
    int32_t *state = nullptr;                   // {token, pos, step, flag, epoch, fault, -, -}
    unsigned long long *qkv_tag = nullptr;      // fused qkv + attention: (tag, value) of the qkv rows
    int32_t *token_log = nullptr, *out_idx = nullptr;
    unsigned *counters = nullptr;
    float *am_val = nullptr, *part = nullptr;
    int32_t *am_idx = nullptr;
    int n_split = 0, use_graph = 1;             // attention splits (0: automatic per context bucket)
    int attn_waves = 4;                         // waves per attention block (4 or 8)
    int attn_step = 4;                          // 4: k_attn_step (4 waves per block); 0: k_attn_decode
    int attn_fuse = 1;                          // 1: the qkv matvec and k_attn_step in one launch
    int64_t epochs = 0;                         // steps since the tags were last cleared
    unsigned long long *stamps = nullptr;       // profiling build: phase stamps of the fused launch
    // one captured decode step per context bucket (the attention's static
    // partition is sized for the bucket); keyed by the bucket's capacity
    std::map<int64_t, hipGraphExec_t> graphs;
    int64_t step_pos = 0;                       // position of the next step to enqueue
    int32_t host_state[4] = {0, 0, 0, 0};
    PrefillBufs pf;
    DevBuf head_out;                            // prefill_logits / prefill_argmax outputs, kept between calls
    DevBuf gemm_ws;                             // the prefill GEMMs' split-K partials (2 x rows x 1024 f32)
    std::vector<void *> allocs;
};

// Grows the KV cache (doubling, decoder.rs:199-231) so that it holds `need`
// positions; nothing happens when it already does.
int decoder_reserve(qasr_decoder *d, int64_t need);
// lm_head (nullable): a separate bf16 [lm_rows, hidden] host head, packed as
// the int8 decode head instead of the tied embedding (decoder.rs:143-157)
int decoder_build(qasr_decoder *d, const qasr_dec_weights *w, const uint16_t *lm_head, int64_t lm_rows);
// qasr_hip_decoder_load with an optional separate head (bf16 [lm_rows, hidden])
int decoder_load_impl(qasr_hip *h, const qasr_dec_config *cfg, const qasr_dec_weights *w, const uint16_t *lm_head,
                      int64_t lm_rows, int round_mode, int64_t max_seq, int kv_bf16, qasr_decoder **out);
// enqueue one decode step; only_kind >= 0 launches only the kernels of that
// kind (0 norm+qkv, 1 attention, 2 o_proj, 3 norm+gate_up, 4 down, 5 LM head)
// The step is enqueued for position d->step_pos (the caller advances it).
int decoder_enqueue_step(qasr_decoder *d, bool embed_mode, int only_kind = -1);
// context capacity of the bucket holding a context of L positions
int64_t decoder_ctx_cap(const qasr_decoder *d, int64_t L);
void decoder_free_prefill(qasr_decoder *d);
int decoder_prefill_dev(qasr_decoder *d, const float *emb_dev, int64_t S);

// One sequence of a multi-sequence prefill: n rows (device f32 [n][hidden])
// at positions [start, start + n) of the KV view (kc, vc: layer 0's cache of
// this sequence; layer_elems: the stride between layers; head_stride: between
// KV heads, max_seq x head_dim).
struct PrefillSeg {
    const float *rows = nullptr;
    int64_t n = 0, start = 0;
    float *kc = nullptr, *vc = nullptr;
    int64_t layer_elems = 0, head_stride = 0, cap = 0;
};
// decoder_prefill over several sequences at once: the GEMMs, RMSNorm and
// SwiGLU run over all rows together, the q/k norm + RoPE + KV write and the
// causal attention per sequence; every row gets the bits a prefill of its own
// sequence alone would give.
int decoder_prefill_segments(qasr_decoder *d, const PrefillSeg *segs, int n_seg);
int decoder_run_embed_step(qasr_decoder *d);
int decoder_run_embed_steps(qasr_decoder *d, int64_t n);
// host -> device decode state {token, pos = d->len, 0, 0} and the RoPE rows of pos
int decoder_set_state(qasr_decoder *d, int32_t token);
// after the caller's synchronisation: QASR_ERR_HIP when a fused qkv + attention
// launch of the steps since the last check gave up waiting for its qkv values
// (those steps' tokens are not valid); clears the flag
int decoder_fault_check(qasr_decoder *d);
