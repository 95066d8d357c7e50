/*
 * rn_lanes.c — CPU oracle for the multi-lane hyper-connection of Needle 3
 * (crates/model/src/lanes.rs) (test infrastructure, see rn_oracle.h; never the
 * product path). sigmoid (ops.rs:68-71) and sinkhorn_in_place (ops.rs:198-217)
 * call the C library's expf, as the reference's f32::exp does.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rn_oracle.h"

#define RO_SINKHORN_ITERATIONS 20  /* lanes.rs:6 */
#define RO_PRE_LANE_BOOST 8.0f     /* lanes.rs:7 */
#define RO_PRE_LANE_FLOOR -4.0f    /* lanes.rs:8 */
#define RO_POST_LANE_FLOOR -4.0f   /* lanes.rs:9 */

/* ops.rs:60-66 */
void ro_unit_rms(const float* x, int n, float* out) {
    const float inverse = 1.0f / sqrtf(ro_sum_of_squares(x, n) / (float)n + 1e-6f);
    for (int i = 0; i < n; ++i) out[i] = x[i] * inverse;
}

static float sigmoid_libm(float v) { return 1.0f / (1.0f + expf(-v)); }

/* ops.rs:198-217 (row sums and column sums fold from -0.0, as Iterator::sum) */
void ro_sinkhorn(float* m, int size, int iterations) {
    for (int r = 0; r < size; ++r) {
        float peak = -INFINITY;
        for (int c = 0; c < size; ++c) peak = fmaxf(peak, m[r * size + c]);
        for (int c = 0; c < size; ++c) m[r * size + c] = expf(m[r * size + c] - peak);
    }
    for (int it = 0; it < iterations; ++it) {
        for (int r = 0; r < size; ++r) {
            float total = -0.0f;
            for (int c = 0; c < size; ++c) total = total + m[r * size + c];
            const float inverse = 1.0f / fmaxf(total, 1.17549435e-38f);
            for (int c = 0; c < size; ++c) m[r * size + c] = m[r * size + c] * inverse;
        }
        for (int c = 0; c < size; ++c) {
            float total = -0.0f;
            for (int r = 0; r < size; ++r) total = total + m[r * size + c];
            const float inverse = 1.0f / fmaxf(total, 1.17549435e-38f);
            for (int r = 0; r < size; ++r) m[r * size + c] = m[r * size + c] * inverse;
        }
    }
}

/* lanes.rs:48-84 after the three products: pre/post [lanes], residual
 * [lanes*lanes] hold the rows layer*lanes.. of phi_pre/phi_post and
 * layer*lanes*lanes.. of phi_res; input [width] and post, residual updated. */
void ro_lanes_route_tail(int lanes, int width, int layer, int slot, const float* a_pre, const float* a_post,
                         const float* a_res, const float* b_pre, const float* b_post, const float* b_res,
                         const float* stream, const float* pre, float* post, float* residual, float* input) {
    const int own = slot % lanes;
    for (int i = 0; i < width; ++i) input[i] = 0.0f;
    for (int lane = 0; lane < lanes; ++lane) {
        const float pre_offset = lane == own ? RO_PRE_LANE_BOOST + RO_PRE_LANE_FLOOR : RO_PRE_LANE_FLOOR;
        const float gate = sigmoid_libm(a_pre[layer] * pre[lane] + b_pre[layer * lanes + lane] + pre_offset);
        for (int i = 0; i < width; ++i) input[i] = input[i] + gate * stream[lane * width + i];
        const float post_offset = lane == own ? 0.0f : RO_POST_LANE_FLOOR;
        post[lane] = 2.0f * sigmoid_libm(a_post[layer] * post[lane] + b_post[layer * lanes + lane] + post_offset);
    }
    const int base = layer * lanes * lanes;
    for (int i = 0; i < lanes * lanes; ++i) residual[i] = a_res[layer] * residual[i] + b_res[base + i];
    ro_sinkhorn(residual, lanes, RO_SINKHORN_ITERATIONS);
}

/* lanes.rs:86-98 */
void ro_lanes_combine(int lanes, int width, const float* post, const float* residual, const float* stream,
                      const float* delta, float* next) {
    for (int lane = 0; lane < lanes; ++lane) {
        float* out = next + (size_t)lane * width;
        for (int i = 0; i < width; ++i) out[i] = 0.0f;
        for (int source = 0; source < lanes; ++source) {
            const float weight = residual[lane * lanes + source];
            for (int i = 0; i < width; ++i) out[i] = out[i] + weight * stream[(size_t)source * width + i];
        }
        for (int i = 0; i < width; ++i) out[i] = out[i] + post[lane] * delta[i];
    }
}
