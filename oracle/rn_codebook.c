/*
 * rn_codebook.c — CPU oracle for the codebook weight format (test
 * infrastructure, see rn_oracle.h; never the product path).
 *
 * A codebook-quantised [rows][columns] matrix (docs/format.md "Codebook-quantised
 * matrices"; cact record.rs:57-84) pads columns to a multiple of the group size.
 * Its blob holds the packed indices, least-significant bits first
 * (rows x padded x index_bits / 8 bytes), then one fp16 L2 norm per
 * (row, group). Group g of a row is (codebook[idx] * norm) . H with H the
 * normalised Walsh-Hadamard matrix of the group size.
 *
 * The product follows the reference's integer path (the one aarch64 takes):
 *   - the input is rotated group by group (walsh.rs:41-80, matrix.rs:123-128)
 *     and quantised per group to int8 with clamp +-127 (neon.rs:22-106,
 *     panel.rs:52-66);
 *   - the codebook levels become an int8 table with one scale
 *     (IntegerLevels, neon.rs:108-124);
 *   - the exact int32 group sum of table[idx] * code, then per group in order
 *       2-bit (panel.rs:184-188):     total = fmaf(acc, (norm * lscale) * xs, total)
 *       4-bit, ternary (neon.rs:158,180): total = total + (((acc * norm) * lscale) * xs)
 *     (matrix.rs:113-121, 205-214: 2-bit matrices take the panel path, 4-bit
 *     and ternary ones the plane path).
 * 1-bit and 3-bit matrices have no integer path in the reference
 * (matrix.rs:559-563: integer levels for 2 and 4 bits only) and are not
 * restated here.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rn_oracle.h"

/* walsh.rs:41-76: radix-2 butterflies with spans 1, 2, 4, ... (the first two
 * fused into the quad stage, which is the same sums), low = a + b, high = a - b,
 * then every value times 1 / sqrt(n) rounded to float. */
void ro_walsh_transform(float* v, int n) {
    int span = 1;
    if (n >= 4) {
        for (int q = 0; q < n; q += 4) {
            const float a = v[q], b = v[q + 1], c = v[q + 2], d = v[q + 3];
            const float low_sum = a + b, low_difference = a - b;
            const float high_sum = c + d, high_difference = c - d;
            v[q] = low_sum + high_sum;
            v[q + 1] = low_difference + high_difference;
            v[q + 2] = low_sum - high_sum;
            v[q + 3] = low_difference - high_difference;
        }
        span = 4;
    }
    for (; span < n; span *= 2)
        for (int block = 0; block < n; block += 2 * span)
            for (int i = block; i < block + span; ++i) {
                const float a = v[i], b = v[i + span];
                v[i] = a + b;
                v[i + span] = a - b;
            }
    const float scale = 1.0f / sqrtf((float)n);
    for (int i = 0; i < n; ++i) v[i] = v[i] * scale;
}

/* matrix.rs:123-138 and walsh.rs:78-80: copy `columns` values, zero-pad to
 * `padded`, rotate each group. */
void ro_codebook_prepare(const float* x, int columns, int padded, int group, float* rotated) {
    memcpy(rotated, x, (size_t)columns * sizeof(float));
    for (int i = columns; i < padded; ++i) rotated[i] = 0.0f;
    for (int g = 0; g < padded; g += group) ro_walsh_transform(rotated + g, group);
}

/* codebook.rs:12-43 and matrix.rs:499-508: the float levels of a bit width,
 * padded with zeros to 16. Returns the count of levels (2^index_bits), 0 for an
 * unknown width. */
int ro_codebook_levels(const float* codebook, int bits, int group, float levels[16]) {
    for (int i = 0; i < 16; ++i) levels[i] = 0.0f;
    switch (bits) {
        case 1: {
            const float level = sqrtf(2.0f / 3.14159265358979323846f) / sqrtf((float)group);
            levels[0] = -level;
            levels[1] = level;
            return 2;
        }
        case 2: memcpy(levels, codebook, 4 * sizeof(float)); return 4;
        case 3: memcpy(levels, codebook + 4, 8 * sizeof(float)); return 8;
        case 4: memcpy(levels, codebook + 12, 16 * sizeof(float)); return 16;
        case 5: {
            const float level = 1.2240064f / sqrtf((float)group);
            levels[1] = level;
            levels[3] = -level;
            return 4;
        }
        default: return 0;
    }
}

/* neon.rs:114-124: scale = peak / 127 (1.0 for a zero peak), table entry =
 * level / scale rounded half away from zero (Rust f32::round). */
float ro_integer_levels(const float levels[16], int count, int8_t table[16]) {
    float peak = 0.0f;
    for (int i = 0; i < count; ++i) peak = fmaxf(peak, fabsf(levels[i]));
    const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
    for (int i = 0; i < 16; ++i) table[i] = 0;
    for (int i = 0; i < count; ++i) table[i] = (int8_t)roundf(levels[i] / scale);
    return scale;
}

/* panel.rs:52-66 / neon.rs:63-106: per group, scale = peak / 127 (1.0 for a
 * zero peak) and code = round-half-even(x / scale) clamped to +-127, NaN -> 0.
 * codes in natural order. */
void ro_group_codes(const float* rotated, int n, int group, int8_t* codes, float* scales) {
    for (int g = 0; g < n / group; ++g) {
        const float* s = rotated + (size_t)g * group;
        const float peak = ro_peak_magnitude(s, group);
        const float scale = peak > 0.0f ? peak / 127.0f : 1.0f;
        scales[g] = scale;
        for (int i = 0; i < group; ++i) {
            float q = rintf(s[i] / scale);
            q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
            codes[(size_t)g * group + i] = q != q ? 0 : (int8_t)q;
        }
    }
}

/* record.rs:66-72: the index width in the blob (ternary crumbs are 2 bits) */
static int index_bits(int bits) { return bits == 5 ? 2 : bits; }

/* matrix.rs:623-631: the index of element e of a packed row (LSB first) */
static int code_at(const uint8_t* row, int e, int ib) {
    const int bit = e * ib;
    return (row[bit / 8] >> (bit % 8)) & ((1 << ib) - 1);
}

/* y[t][rows] for `count` inputs given as per-group codes [t][padded] and scales
 * [t][padded/group]; acc (nullable) [t][rows][padded/group]. */
void ro_codebook_product(const uint8_t* packed, const uint16_t* norms, int rows, int padded, int group,
                         int bits, const int8_t table[16], float lscale, const int8_t* xcodes,
                         const float* xscales, int count, float* y, int32_t* acc) {
    const int ib = index_bits(bits), groups = padded / group;
    const size_t row_bytes = (size_t)padded * ib / 8;
#pragma omp parallel for schedule(static) if ((size_t)rows * padded * count >= (1u << 22))
    for (int r = 0; r < rows; ++r) {
        const uint8_t* row = packed + (size_t)r * row_bytes;
        for (int t = 0; t < count; ++t) {
            const int8_t* xc = xcodes + (size_t)t * padded;
            const float* xs = xscales + (size_t)t * groups;
            float total = 0.0f;
            for (int g = 0; g < groups; ++g) {
                int32_t a = 0;
                for (int i = 0; i < group; ++i) {
                    const int e = g * group + i;
                    a += (int32_t)table[code_at(row, e, ib)] * (int32_t)xc[e];
                }
                if (acc) acc[((size_t)t * rows + r) * groups + g] = a;
                const float norm = ro_f16_to_f32(norms[(size_t)r * groups + g]);
                if (bits == 2)
                    total = fmaf((float)a, (norm * lscale) * xs[g], total);
                else
                    total = total + ((((float)a * norm) * lscale) * xs[g]);
            }
            y[(size_t)t * rows + r] = total;
        }
    }
}

/* matrix.rs:140-153: out[columns] = per group (level[idx] * norm) then the
 * Walsh-Hadamard transform of the group, truncated to `columns`. */
void ro_codebook_dequantise_row(const uint8_t* packed, const uint16_t* norms, int padded, int columns,
                                int group, int bits, const float levels[16], int row, float* out) {
    const int ib = index_bits(bits), groups = padded / group;
    const uint8_t* r = packed + (size_t)row * padded * ib / 8;
    float* full = (float*)malloc((size_t)padded * sizeof(float));
    for (int g = 0; g < groups; ++g) {
        const float norm = ro_f16_to_f32(norms[(size_t)row * groups + g]);
        for (int i = 0; i < group; ++i) full[g * group + i] = levels[code_at(r, g * group + i, ib)] * norm;
        ro_walsh_transform(full + g * group, group);
    }
    memcpy(out, full, (size_t)columns * sizeof(float));
    free(full);
}
