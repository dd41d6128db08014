/*
 * TEST INFRASTRUCTURE ONLY -- the checker, never the product. Only tests/, the smoke check of
 * __graft_entry__.py and the CPU-baseline leg of bench.py may load this library.
 *
 * Exact attention in double precision, one query row at a time, over fp16 inputs given as
 * IEEE binary16 bit patterns. Restates the reference's fp64 CPU references:
 *   tests/cpp/test_flash_fwd.cu:115-152  (cpu_attention: all rows)
 *   csrc/dev/main.cu:31-63               (reference_row: one row)
 * per row i of head bh: s_j = (q_i . k_j) * scale for the visible keys j (j <= i when causal),
 * p_j = exp(s_j - max_j s_j) / sum_j exp(s_j - max), o_i = sum_j p_j v_j.
 * Unlike the reference's versions the scale is a parameter (they fix 1/sqrt(d)), so the
 * custom-scale path of the binding (csrc/bindings.cpp:55-56) can be checked as well.
 * oracle_lse_rows gives the same rows' log-sum-exp, max_j s_j + log(sum_j exp(s_j - max)):
 * the reference computes it only implicitly (its kernel keeps m and l, flash_fwd.cu:526-560).
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

/* binary16 -> double from the format's definition: 1 sign bit, 5 exponent bits (bias 15),
 * 10 fraction bits; exponent 0 = subnormal (no implicit 1), 31 = inf/nan. */
double oracle_half_to_double(uint16_t h) {
    const int sign = (h >> 15) & 1;
    const int exp = (h >> 10) & 0x1f;
    const int frac = h & 0x3ff;
    double mag;
    if (exp == 0) {
        mag = ldexp((double)frac, -24); /* frac * 2^-10 * 2^-14 */
    } else if (exp == 31) {
        mag = frac ? NAN : INFINITY;
    } else {
        mag = ldexp((double)(frac | 0x400), exp - 25); /* (1 + frac/1024) * 2^(exp-15) */
    }
    return sign ? -mag : mag;
}

/* Attention rows rows[0..n_rows) of head `bh` of [B*H, n, d] tensors. out: n_rows * d doubles.
 * Returns 0, or -1 on bad arguments / allocation failure. */
int oracle_attention_rows(const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t bh,
                          int64_t n, int64_t d, double scale, int causal, const int64_t* rows,
                          int64_t n_rows, double* out) {
    if (n <= 0 || d <= 0 || n_rows < 0) return -1;
    const size_t base = (size_t)bh * (size_t)n * (size_t)d;
    double* s = (double*)malloc((size_t)n * sizeof(double));
    double* qi = (double*)malloc((size_t)d * sizeof(double));
    if (s == NULL || qi == NULL) {
        free(s);
        free(qi);
        return -1;
    }
    for (int64_t r = 0; r < n_rows; ++r) {
        const int64_t i = rows[r];
        if (i < 0 || i >= n) {
            free(s);
            free(qi);
            return -1;
        }
        const int64_t kv_end = causal ? i + 1 : n;
        for (int64_t c = 0; c < d; ++c) qi[c] = oracle_half_to_double(q[base + (size_t)(i * d + c)]);
        double mx = -INFINITY;
        for (int64_t j = 0; j < kv_end; ++j) {
            const uint16_t* kj = k + base + (size_t)(j * d);
            double dot = 0.0;
            for (int64_t c = 0; c < d; ++c) dot += qi[c] * oracle_half_to_double(kj[c]);
            s[j] = dot * scale;
            if (s[j] > mx) mx = s[j];
        }
        double sum = 0.0;
        for (int64_t j = 0; j < kv_end; ++j) {
            s[j] = exp(s[j] - mx);
            sum += s[j];
        }
        double* o = out + (size_t)(r * d);
        for (int64_t c = 0; c < d; ++c) o[c] = 0.0;
        for (int64_t j = 0; j < kv_end; ++j) {
            const double p = s[j] / sum;
            const uint16_t* vj = v + base + (size_t)(j * d);
            for (int64_t c = 0; c < d; ++c) o[c] += p * oracle_half_to_double(vj[c]);
        }
    }
    free(s);
    free(qi);
    return 0;
}

/* Natural-log log-sum-exp of the scaled scores of rows rows[0..n_rows) of head `bh`:
 * out[r] = max_j s_j + log(sum_j exp(s_j - max_j s_j)) over the visible keys. Returns 0 or -1. */
int oracle_lse_rows(const uint16_t* q, const uint16_t* k, int64_t bh, int64_t n, int64_t d,
                    double scale, int causal, const int64_t* rows, int64_t n_rows, double* out) {
    if (n <= 0 || d <= 0 || n_rows < 0) return -1;
    const size_t base = (size_t)bh * (size_t)n * (size_t)d;
    double* s = (double*)malloc((size_t)n * sizeof(double));
    if (s == NULL) return -1;
    for (int64_t r = 0; r < n_rows; ++r) {
        const int64_t i = rows[r];
        if (i < 0 || i >= n) {
            free(s);
            return -1;
        }
        const int64_t kv_end = causal ? i + 1 : n;
        double mx = -INFINITY;
        for (int64_t j = 0; j < kv_end; ++j) {
            double dot = 0.0;
            for (int64_t c = 0; c < d; ++c) {
                dot += oracle_half_to_double(q[base + (size_t)(i * d + c)]) *
                       oracle_half_to_double(k[base + (size_t)(j * d + c)]);
            }
            s[j] = dot * scale;
            if (s[j] > mx) mx = s[j];
        }
        double sum = 0.0;
        for (int64_t j = 0; j < kv_end; ++j) sum += exp(s[j] - mx);
        out[r] = mx + log(sum);
    }
    free(s);
    return 0;
}
