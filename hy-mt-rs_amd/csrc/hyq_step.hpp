// Decode-step glue launchers (kernels in hyq_step.hip).
#pragma once

#include <stdint.h>

#include "hyq_internal.hpp"

namespace hyq {

// Device-resident step state: the position of the token being decoded and the
// number of tokens generated so far (index into the history buffer).
struct StepState {
    int pos;
    int step;
    int history_cap;
    int pad;
};

int launch_embed_row(int fmt, WView w, int cols, const int *token, float *out, void *stream);
int launch_rms_norm_q8(const float *x, const float *w, int n, float eps, float *y, int8_t *q,
                       float *s, int32_t *s16, int32_t *s32, int32_t *s256, void *stream);
int launch_rope_norm_kv(float *q, const float *k, const float *v, const float *qn,
                        const float *kn, const float *freq, const int *pos, int heads, int kvh,
                        int dim, float eps, float *kcache, float *vcache, void *stream);
int attention_splits(int context);
int launch_attention(const float *q, const float *kcache, const float *vcache, const int *pos,
                     int context, int heads, int kvh, float *part, float *out, int8_t *qq,
                     float *s, int32_t *s16, int32_t *s32, int32_t *s256, void *stream);
int argmax_partials(int n);
int launch_argmax(const float *x, int n, float *pv, int *pi, int *token, StepState *st,
                  int *history, void *stream);

} // namespace hyq
