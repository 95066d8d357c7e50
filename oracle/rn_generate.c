/*
 * rn_generate.c — CPU oracle for the grammar-constrained choice of the
 * generator (test infrastructure, see rn_oracle.h; never the product path).
 *
 * generator.rs:99-117 picks argmax_allowed(logits, allowed) (falling back to
 * argmax when nothing is allowed) and, while a constraint is active, adds the
 * allowed_statistics of the chosen token to the turn's call probability and
 * minimum allowed mass.
 */
#include <math.h>
#include <stdint.h>

#include "rn_oracle.h"

/* generator.rs:147-155: the first allowed index whose value is greater than
 * every earlier allowed value (a NaN wins only as the first allowed value);
 * -1 when nothing is allowed. */
int32_t ro_argmax_allowed(const float* values, const uint8_t* allowed, int n) {
    int32_t best = -1;
    for (int i = 0; i < n; ++i)
        if (allowed[i] && (best < 0 || values[i] > values[best])) best = i;
    return best;
}

/* generator.rs:182-194 with peak_of (generator.rs:178-180): peaks fold from
 * -inf with f32::max (NaN ignored, as fmaxf); the two totals run sequentially
 * in index order; a disallowed value contributes fast_exp(v - peak_allowed) * 0. */
void ro_allowed_statistics(const float* logits, const uint8_t* allowed, int n, int token, float* probability,
                           float* mass) {
    float peak_all = -INFINITY, peak_allowed = -INFINITY;
    for (int i = 0; i < n; ++i) {
        peak_all = fmaxf(peak_all, logits[i]);
        peak_allowed = fmaxf(peak_allowed, allowed[i] ? logits[i] : -INFINITY);
    }
    float total_all = 0.0f, total_allowed = 0.0f;
    for (int i = 0; i < n; ++i) {
        total_all = total_all + ro_fast_exp(logits[i] - peak_all);
        total_allowed = total_allowed + ro_fast_exp(logits[i] - peak_allowed) * (allowed[i] ? 1.0f : 0.0f);
    }
    *probability = ro_fast_exp(logits[token] - peak_allowed) / total_allowed;
    *mass = (total_allowed * ro_fast_exp(peak_allowed - peak_all)) / total_all;
}
