// Internal entry points of the device-resident audio front end (encoder.cpp)
// used by the other drivers (streaming).
#pragma once
#include <stdint.h>
#include <stddef.h>
#include "model.h"

// samples -> mel frames of mel_spectrogram (audio.rs:273-294; 0 when too short)
int64_t mel_frames_for(int64_t n_samples);
// floats of scratch mel_dev needs for nf frames
size_t mel_scratch_floats(int64_t nf);
// mel_spectrogram on device samples x[ns]; mel [128][frames]
int mel_dev(qasr_encoder *e, const float *x, int64_t ns, float *mel, float *scratch);
// Encoder::forward on a device mel [128][frames]; out [tokens][output_dim]
int encoder_forward_dev(qasr_encoder *e, const float *mel, int64_t frames, float *out, int64_t *n_tok);
// n (<= 64) sequences in one pass; sequence j's rows at out + (T_0 + ... + T_{j-1}) rows
int encoder_forward_multi(qasr_encoder *e, int n, const float *const *mels, const int64_t *frames, float *out,
                          int64_t *tokens);
int64_t encoder_tokens(const qasr_encoder *e, int64_t frames);
int64_t encoder_output_dim(const qasr_encoder *e);
qasr_hip *encoder_handle(const qasr_encoder *e);
// mel_spectrogram of n device signals with their DFT and filterbank GEMMs
// shared; mel[j] [128][frames_j] each
int mel_dev_multi(qasr_encoder *e, int n, const float *const *x, const int64_t *ns, float *const *mel, float *scratch);
size_t mel_multi_scratch_floats(int64_t total_frames, int64_t max_frames);
