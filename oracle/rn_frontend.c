/*
 * rn_frontend.c — CPU oracle for the speech front end (test infrastructure,
 * see rn_oracle.h; never the product path): Frontend::new / log_mel / spread /
 * normalise of crates/whistle/src/frontend.rs.
 *
 * Float operations follow the reference in order (-ffp-contract=off keeps
 * every a*b+c as two roundings): the Hann window and the twiddles from cosf /
 * sinf in float, a radix-2 decimation-in-time FFT after the bit-reversal
 * permutation, power = re*re + im*im, mel rows accumulated bin by bin, ln from
 * the C library (Rust's f32::ln is the platform logf), per-mel sums over frames
 * in frame order (Iterator::sum of f32 starts from -0.0, which differs from
 * +0.0 only for a sum of no values or of negative zeros).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "rn_oracle.h"

#define RO_PI 3.14159265358979323846f
#define RO_FLOOR 5.9604645e-8f           /* frontend.rs:3 */
#define RO_NORMALISER_EPSILON 1e-5f      /* frontend.rs:4 */

/* frontend.rs:32-39: window[n] = 0.5 - 0.5 cos(2 pi n / (window - 1)),
 * twiddle_cos[k] = cos(2 pi k / size), twiddle_sin[k] = -sin(2 pi k / size). */
void ro_frontend_tables(int fft_size, int window, float* win, float* twiddle_cos, float* twiddle_sin) {
    for (int n = 0; n < window; ++n)
        win[n] = 0.5f - 0.5f * cosf(((2.0f * RO_PI) * (float)n) / (float)(window - 1));
    for (int k = 0; k < fft_size / 2; ++k) {
        twiddle_cos[k] = cosf(((2.0f * RO_PI) * (float)k) / (float)fft_size);
        twiddle_sin[k] = -sinf(((2.0f * RO_PI) * (float)k) / (float)fft_size);
    }
}

static unsigned reverse_bits(unsigned i, int bits) {
    unsigned r = 0;
    for (int b = 0; b < bits; ++b) r |= ((i >> b) & 1u) << (bits - 1 - b);
    return r;
}

/* frontend.rs:42-70: bit-reversal swaps, butterflies of span 1, 2, 4, ...,
 * power[bin] for bin <= size/2. real/imaginary are overwritten. */
void ro_power_spectrum(float* real, float* imaginary, int size, const float* twiddle_cos, const float* twiddle_sin,
                       float* power) {
    int bits = 0;
    while ((1 << bits) < size) ++bits;
    for (int i = 0; i < size; ++i) {
        const int t = (int)reverse_bits((unsigned)i, bits);
        if (t > i) {
            float x = real[i]; real[i] = real[t]; real[t] = x;
            x = imaginary[i]; imaginary[i] = imaginary[t]; imaginary[t] = x;
        }
    }
    for (int span = 1; span < size; span *= 2) {
        const int stride = size / (span * 2);
        for (int start = 0; start < size; start += 2 * span)
            for (int offset = 0; offset < span; ++offset) {
                const float c = twiddle_cos[offset * stride], s = twiddle_sin[offset * stride];
                const int a = start + offset, b = a + span;
                const float tr = real[b] * c - imaginary[b] * s;
                const float ti = real[b] * s + imaginary[b] * c;
                real[b] = real[a] - tr;
                imaginary[b] = imaginary[a] - ti;
                real[a] = real[a] + tr;
                imaginary[a] = imaginary[a] + ti;
            }
    }
    for (int bin = 0; bin <= size / 2; ++bin) power[bin] = real[bin] * real[bin] + imaginary[bin] * imaginary[bin];
}

/* frontend.rs:72-102 up to (not including) spread and normalise: data
 * [frames][mels] = ln(mel projection of the power spectrum + FLOOR), frames =
 * n / hop + 1. mel_weights is [fft_size/2 + 1][mels]. Returns frames. */
int ro_log_mel_raw(const float* samples, int n, int mels, int fft_size, int window, int hop,
                   const float* mel_weights, float* data) {
    const int frames = n / hop + 1, half = window / 2, bins = fft_size / 2 + 1;
    float* win = (float*)malloc(sizeof(float) * (size_t)window);
    float* tc = (float*)malloc(sizeof(float) * (size_t)(fft_size / 2));
    float* ts = (float*)malloc(sizeof(float) * (size_t)(fft_size / 2));
    float* re = (float*)malloc(sizeof(float) * (size_t)fft_size);
    float* im = (float*)malloc(sizeof(float) * (size_t)fft_size);
    float* power = (float*)malloc(sizeof(float) * (size_t)bins);
    ro_frontend_tables(fft_size, window, win, tc, ts);
    for (int f = 0; f < frames; ++f) {
        memset(re, 0, sizeof(float) * (size_t)fft_size);
        memset(im, 0, sizeof(float) * (size_t)fft_size);
        for (int p = 0; p < window && p < fft_size; ++p) {
            const long source = (long)f * hop + p - half;
            if (source >= 0 && source < n) re[p] = samples[source] * win[p];
        }
        ro_power_spectrum(re, im, fft_size, tc, ts, power);
        float* row = data + (size_t)f * mels;
        for (int m = 0; m < mels; ++m) row[m] = 0.0f;
        for (int bin = 0; bin < bins; ++bin)
            for (int m = 0; m < mels; ++m) row[m] = row[m] + power[bin] * mel_weights[(size_t)bin * mels + m];
        for (int m = 0; m < mels; ++m) row[m] = logf(row[m] + RO_FLOOR);
    }
    free(win); free(tc); free(ts); free(re); free(im); free(power);
    return frames;
}

/* frontend.rs:104-116 */
float ro_spread(const float* data, int valid, int mels) {
    if (valid < 2) return 0.0f;
    float total = 0.0f;
    for (int m = 0; m < mels; ++m) {
        float sum = -0.0f;  /* Iterator::sum of f32 folds from -0.0 */
        for (int f = 0; f < valid; ++f) sum = sum + data[(size_t)f * mels + m];
        const float mean = sum / (float)valid;
        float sq = -0.0f;
        for (int f = 0; f < valid; ++f) {
            const float d = data[(size_t)f * mels + m] - mean;
            sq = sq + d * d;
        }
        const float variance = sq / (float)(valid - 1);
        total = total + sqrtf(variance);
    }
    return total / (float)mels;
}

/* frontend.rs:118-133: per mel, (x - mean) / (std + 1e-5) over the valid
 * frames (std with denominator max(valid - 1, 1)); frames past valid become 0. */
void ro_normalise(float* data, int frames, int valid, int mels) {
    const float count = (float)(valid > 1 ? valid : 1);
    float denominator = (float)(valid > 1 ? valid : 1) - 1.0f;
    denominator = denominator > 1.0f ? denominator : 1.0f;
    for (int m = 0; m < mels; ++m) {
        float sum = -0.0f;  /* Iterator::sum of f32 folds from -0.0 */
        for (int f = 0; f < valid; ++f) sum = sum + data[(size_t)f * mels + m];
        const float mean = sum / count;
        float sq = -0.0f;
        for (int f = 0; f < valid; ++f) {
            const float d = data[(size_t)f * mels + m] - mean;
            sq = sq + d * d;
        }
        const float variance = sq / denominator;
        const float scale = 1.0f / (sqrtf(variance) + RO_NORMALISER_EPSILON);
        for (int f = 0; f < frames; ++f) {
            float* slot = data + (size_t)f * mels + m;
            *slot = f < valid ? (*slot - mean) * scale : 0.0f;
        }
    }
}

/* Frontend::log_mel (frontend.rs:72-102): data [n / hop + 1][mels]; returns
 * frames; *valid = n / hop; *spread from the un-normalised data. */
int ro_log_mel(const float* samples, int n, int mels, int fft_size, int window, int hop, const float* mel_weights,
               float* data, int* valid, float* spread) {
    const int frames = ro_log_mel_raw(samples, n, mels, fft_size, window, hop, mel_weights, data);
    *valid = n / hop;
    *spread = ro_spread(data, *valid, mels);
    ro_normalise(data, frames, *valid, mels);
    return frames;
}
