/*
 * rn_hadamard.c — CPU oracle for kronecker_apply (ops.rs:143-297), the core of
 * the Hadamard MLP (hadamard.rs:55-107) (test infrastructure, see rn_oracle.h;
 * never the product path).
 *
 * For 32 x 32 factors the reference's aarch64 path (ops.rs:220-297) forms
 * mixed = X . R and out = L^T . mixed with fused multiply-adds: mixed[i][c]
 * accumulates fma(x[i][j], r[j][c], .) for j = 0..31 from 0, and out[k][c]
 * accumulates fma(l[i][k], mixed[i][c], .) for i = 0..31 from 0.
 */
#include <math.h>

#include "rn_oracle.h"

void ro_kronecker_apply_32(const float* input, const float* left, const float* right, float* output) {
    float mixed[32 * 32];
    for (int i = 0; i < 32; ++i)
        for (int c = 0; c < 32; ++c) {
            float acc = 0.0f;
            for (int j = 0; j < 32; ++j) acc = fmaf(right[j * 32 + c], input[i * 32 + j], acc);
            mixed[i * 32 + c] = acc;
        }
    for (int k = 0; k < 32; ++k)
        for (int c = 0; c < 32; ++c) {
            float acc = 0.0f;
            for (int i = 0; i < 32; ++i) acc = fmaf(mixed[i * 32 + c], left[i * 32 + k], acc);
            output[k * 32 + c] = acc;
        }
}
