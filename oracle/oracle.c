/*
 * CPU oracle for the butterfly execution path -- TEST INFRASTRUCTURE ONLY.
 * See oracle.h for the contract; each function cites the reference code it
 * restates. Built with -ffp-contract=off so every float/double operation is
 * rounded exactly where the reference source rounds it.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

static int is_pow2(uint64_t n) { return n != 0 && (n & (n - 1)) == 0; }

static uint32_t log2_exact(uint64_t n) {
    uint32_t log_n = 0;
    while ((UINT64_C(1) << log_n) < n) ++log_n;
    return log_n;
}

static uint64_t reverse_bits(uint64_t index, uint32_t bits) {
    uint64_t result = 0;
    for (uint32_t j = 0; j < bits; ++j, index >>= 1) result = (result << 1) | (index & 1);
    return result;
}

/* ---- row-parallel driver ------------------------------------------------ */

typedef int (*row_fn)(void* context, uint64_t row);

typedef struct {
    row_fn fn;
    void* context;
    uint64_t begin, end;
    int status;
} row_span;

static void* run_span(void* argument) {
    row_span* span = (row_span*)argument;
    for (uint64_t row = span->begin; row < span->end && span->status == 0; ++row)
        span->status = span->fn(span->context, row);
    return NULL;
}

static int for_rows(uint64_t rows, int threads, row_fn fn, void* context) {
    if (threads <= 1 || rows <= 1) {
        row_span span = {fn, context, 0, rows, 0};
        run_span(&span);
        return span.status;
    }
    if ((uint64_t)threads > rows) threads = (int)rows;
    pthread_t* ids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
    row_span* spans = (row_span*)calloc((size_t)threads, sizeof(row_span));
    if (!ids || !spans) {
        free(ids);
        free(spans);
        return -1;
    }
    int status = 0, started = 0;
    for (int t = 0; t < threads; ++t) {
        spans[t].fn = fn;
        spans[t].context = context;
        spans[t].begin = rows * (uint64_t)t / (uint64_t)threads;
        spans[t].end = rows * (uint64_t)(t + 1) / (uint64_t)threads;
        if (pthread_create(&ids[t], NULL, run_span, &spans[t]) != 0) {
            status = -1;
            break;
        }
        ++started;
    }
    for (int t = 0; t < started; ++t) {
        pthread_join(ids[t], NULL);
        if (spans[t].status) status = spans[t].status;
    }
    free(ids);
    free(spans);
    return status;
}

/* ---- FWHT: src/butterfly_reference.cpp:349-369 -------------------------- */

int cbo_fwht_f32(float* values, uint64_t n, int inverse, int normalize) {
    if (!values || !is_pow2(n)) return -1;
    for (uint64_t half = 1; half < n; half <<= 1) {
        for (uint64_t base = 0; base < n; base += 2 * half) {
            for (uint64_t offset = 0; offset < half; ++offset) {
                const float left = values[base + offset];
                const float right = values[base + half + offset];
                values[base + offset] = left + right;
                values[base + half + offset] = left - right;
            }
        }
    }
    if (inverse && normalize) {
        const float scale = 1.0f / (float)n;
        for (uint64_t i = 0; i < n; ++i) values[i] *= scale;
    }
    return 0;
}

typedef struct {
    float* values;
    uint64_t n;
    int inverse, normalize;
} fwht_ctx;

static int fwht_row(void* context, uint64_t row) {
    fwht_ctx* c = (fwht_ctx*)context;
    return cbo_fwht_f32(c->values + row * c->n, c->n, c->inverse, c->normalize);
}

int cbo_fwht_f32_batch(float* values, uint64_t n, uint64_t batch, int inverse,
                       int normalize, int threads) {
    if (!values || !is_pow2(n)) return -1;
    fwht_ctx c = {values, n, inverse, normalize};
    return for_rows(batch, threads, fwht_row, &c);
}

/* ---- binary16 conversions (IEEE 754-2008 binary16, RNE) ----------------- */

uint16_t cbo_f32_to_f16_rne(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof x);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t exponent = (x >> 23) & 0xffu;
    const uint32_t mantissa = x & 0x7fffffu;
    if (exponent == 0xffu) /* inf stays inf; NaN stays a quiet NaN */
        return (uint16_t)(sign | 0x7c00u | (mantissa ? (0x200u | (mantissa >> 13)) : 0u));
    const int e = (int)exponent - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e >= 1) {
        uint32_t h = ((uint32_t)e << 10) | (mantissa >> 13);
        const uint32_t rest = mantissa & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h; /* a carry may reach inf */
        return (uint16_t)(sign | h);
    }
    if (exponent == 0) return sign; /* f32 zero/subnormal is far below 2^-25 */
    const uint32_t m = mantissa | 0x800000u;
    const int shift = 14 - e; /* value = m * 2^(e-14) half-subnormal units */
    if (shift > 24) return sign;
    uint32_t h = m >> shift;
    const uint32_t rest = m & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rest > halfway || (rest == halfway && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float cbo_f16_to_f32(uint16_t bits) {
    const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    const uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
    uint32_t mantissa = (uint32_t)bits & 0x3ffu;
    uint32_t x;
    if (exponent == 0x1fu) {
        x = sign | 0x7f800000u | (mantissa << 13);
    } else if (exponent != 0) {
        x = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    } else if (mantissa == 0) {
        x = sign;
    } else { /* subnormal: normalise */
        uint32_t e = 113u;
        while ((mantissa & 0x400u) == 0) {
            mantissa <<= 1;
            --e;
        }
        x = sign | (e << 23) | ((mantissa & 0x3ffu) << 13);
    }
    float value;
    memcpy(&value, &x, sizeof value);
    return value;
}

/* ---- FP16 final storage: src/butterfly.cu:1882-1897 and :53-68 ---------- */

typedef struct {
    const uint16_t* input;
    uint16_t* output;
    uint64_t n;
    float scale;
    int inverse, normalize;
} fwht16_ctx;

static int fwht16_row(void* context, uint64_t row) {
    fwht16_ctx* c = (fwht16_ctx*)context;
    float* work = (float*)malloc(c->n * sizeof(float));
    if (!work) return -1;
    const uint16_t* in = c->input + row * c->n;
    uint16_t* out = c->output + row * c->n;
    for (uint64_t i = 0; i < c->n; ++i) work[i] = cbo_f16_to_f32(in[i]); /* widen */
    int status = cbo_fwht_f32(work, c->n, c->inverse, c->normalize);  /* FP32 plan */
    for (uint64_t i = 0; i < c->n; ++i) out[i] = cbo_f32_to_f16_rne(work[i] * c->scale); /* narrow */
    free(work);
    return status;
}

int cbo_fwht_f16_final_batch(const uint16_t* input, uint16_t* output,
                             uint64_t n, uint64_t batch, float scale,
                             int inverse, int normalize, int threads) {
    if (!input || !output || !is_pow2(n)) return -1;
    fwht16_ctx c = {input, output, n, scale, inverse, normalize};
    return for_rows(batch, threads, fwht16_row, &c);
}

/* ---- complex FFT: src/butterfly_reference.cpp:392-433 ------------------- */

int cbo_fft_c64(float* values, uint64_t n, int inverse, int normalize) {
    if (!values || !is_pow2(n)) return -1;
    uint64_t reversed = 0;
    for (uint64_t index = 1; index < n; ++index) {
        uint64_t bit = n >> 1;
        while ((reversed & bit) != 0) {
            reversed ^= bit;
            bit >>= 1;
        }
        reversed ^= bit;
        if (index < reversed) {
            const float re = values[2 * index], im = values[2 * index + 1];
            values[2 * index] = values[2 * reversed];
            values[2 * index + 1] = values[2 * reversed + 1];
            values[2 * reversed] = re;
            values[2 * reversed + 1] = im;
        }
    }
    const double kPi = 3.141592653589793238462643383279502884;
    for (uint64_t half = 1; half < n; half <<= 1) {
        for (uint64_t base = 0; base < n; base += 2 * half) {
            for (uint64_t offset = 0; offset < half; ++offset) {
                const double direction = inverse ? 1.0 : -1.0;
                const double angle = direction * kPi * (double)offset / (double)half;
                const double wr = cos(angle);
                const double wi = sin(angle);
                float* a = values + 2 * (base + offset);
                float* b = values + 2 * (base + half + offset);
                const float ar = a[0], ai = a[1], br = b[0], bi = b[1];
                const float vr = (float)((double)br * wr - (double)bi * wi);
                const float vi = (float)((double)br * wi + (double)bi * wr);
                a[0] = ar + vr;
                a[1] = ai + vi;
                b[0] = ar - vr;
                b[1] = ai - vi;
            }
        }
    }
    if (inverse && normalize) {
        const float scale = 1.0f / (float)n;
        for (uint64_t i = 0; i < 2 * n; ++i) values[i] *= scale;
    }
    return 0;
}

typedef struct {
    float* values;
    uint64_t n;
    int inverse, normalize;
} fft_ctx;

static int fft_row(void* context, uint64_t row) {
    fft_ctx* c = (fft_ctx*)context;
    return cbo_fft_c64(c->values + 2 * row * c->n, c->n, c->inverse, c->normalize);
}

int cbo_fft_c64_batch(float* values, uint64_t n, uint64_t batch, int inverse,
                      int normalize, int threads) {
    if (!values || !is_pow2(n)) return -1;
    fft_ctx c = {values, n, inverse, normalize};
    return for_rows(batch, threads, fft_row, &c);
}

/* ---- modular arithmetic: src/reference.cpp:11-13, 506-582 --------------- */

uint64_t cbo_mod_mul(uint64_t a, uint64_t b, uint64_t q) {
    return (uint64_t)(((u128)a * b) % q);
}

uint64_t cbo_mod_pow(uint64_t base, uint64_t exponent, uint64_t q) {
    if (q < 2) return 0;
    uint64_t result = 1;
    base %= q;
    while (exponent != 0) {
        if (exponent & 1u) result = cbo_mod_mul(result, base, q);
        base = cbo_mod_mul(base, base, q);
        exponent >>= 1;
    }
    return result;
}

int cbo_is_prime(uint64_t value) {
    if (value < 2) return 0;
    static const uint64_t small[12] = {2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37};
    for (int i = 0; i < 12; ++i)
        if (value % small[i] == 0) return value == small[i];
    uint64_t odd = value - 1;
    uint32_t twos = 0;
    while ((odd & 1u) == 0) {
        odd >>= 1;
        ++twos;
    }
    static const uint64_t witnesses[7] = {2, 325, 9375, 28178, 450775, 9780504, 1795265022};
    for (int w = 0; w < 7; ++w) {
        if (witnesses[w] % value == 0) continue;
        uint64_t x = cbo_mod_pow(witnesses[w], odd, value);
        if (x == 1 || x == value - 1) continue;
        int probable = 0;
        for (uint32_t round = 1; round < twos; ++round) {
            x = cbo_mod_mul(x, x, value);
            if (x == value - 1) {
                probable = 1;
                break;
            }
        }
        if (!probable) return 0;
    }
    return 1;
}

uint64_t cbo_find_primitive_root(uint32_t log_n, uint64_t q) {
    if (log_n == 0 || log_n >= 63 || !cbo_is_prime(q)) return 0;
    const uint64_t n = UINT64_C(1) << log_n;
    if ((q - 1) % n != 0) return 0;
    for (uint64_t candidate = 2; candidate < (UINT64_C(1) << 20); ++candidate) {
        const uint64_t root = cbo_mod_pow(candidate, (q - 1) / n, q);
        if (cbo_mod_pow(root, n, q) == 1 && cbo_mod_pow(root, n >> 1, q) != 1) return root;
    }
    return 0;
}

/* benchmarks/crypto_ntt/crypto_ntt_bench.cu:273-290 */
uint64_t cbo_find_psi(uint32_t log_n, uint64_t q, uint64_t root) {
    if (log_n >= 62) return 0;
    const uint64_t default_psi = cbo_find_primitive_root(log_n + 1, q);
    if (default_psi != 0 && cbo_mod_mul(default_psi, default_psi, q) == root) return default_psi;
    const uint64_t order = UINT64_C(1) << (log_n + 1);
    if ((q - 1) % order != 0) return 0;
    for (uint64_t candidate = 2; candidate < (UINT64_C(1) << 20); ++candidate) {
        const uint64_t psi = cbo_mod_pow(candidate, (q - 1) / order, q);
        if (cbo_mod_pow(psi, order, q) == 1 && cbo_mod_pow(psi, order >> 1, q) != 1 &&
            cbo_mod_mul(psi, psi, q) == root)
            return psi;
    }
    return 0;
}

/* ---- cyclic NTT: src/reference.cpp:584-630 ------------------------------ */

/* Radix-2 DIT after a bit-reversal permutation with an explicit root; shared
 * by reference_ntt and by independent_ntt's n > 256 branch
 * (crypto_ntt_bench.cu:478-507), which are the same loop nest. */
static void dit_with_root(uint64_t* values, uint64_t n, uint64_t q, uint64_t root) {
    const uint32_t log_n = log2_exact(n);
    for (uint64_t i = 0; i < n; ++i) {
        const uint64_t r = reverse_bits(i, log_n);
        if (i < r) {
            const uint64_t t = values[i];
            values[i] = values[r];
            values[r] = t;
        }
    }
    for (uint64_t length = 2; length <= n; length <<= 1) {
        const uint64_t half = length >> 1;
        const uint64_t step = cbo_mod_pow(root, n / length, q);
        for (uint64_t start = 0; start < n; start += length) {
            uint64_t omega = 1;
            for (uint64_t offset = 0; offset < half; ++offset) {
                const uint64_t left = start + offset;
                const uint64_t u = values[left];
                const uint64_t v = cbo_mod_mul(values[left + half], omega, q);
                const uint64_t sum = u + v;
                values[left] = sum >= q ? sum - q : sum;
                values[left + half] = u >= v ? u - v : q + u - v;
                omega = cbo_mod_mul(omega, step, q);
            }
        }
    }
}

int cbo_ntt_cyclic(uint64_t* values, uint64_t n, uint64_t q, int inverse) {
    if (!values || n < 2 || !is_pow2(n) || q >= (UINT64_C(1) << 63)) return -1;
    uint64_t root = cbo_find_primitive_root(log2_exact(n), q);
    if (root == 0) return -1;
    if (inverse) root = cbo_mod_pow(root, q - 2, q);
    for (uint64_t i = 0; i < n; ++i) values[i] %= q;
    dit_with_root(values, n, q, root);
    if (inverse) {
        const uint64_t inverse_n = cbo_mod_pow(n, q - 2, q);
        for (uint64_t i = 0; i < n; ++i) values[i] = cbo_mod_mul(values[i], inverse_n, q);
    }
    return 0;
}

typedef struct {
    uint64_t* values;
    uint64_t n, q;
    int inverse;
} ntt_ctx;

static int ntt_row(void* context, uint64_t row) {
    ntt_ctx* c = (ntt_ctx*)context;
    return cbo_ntt_cyclic(c->values + row * c->n, c->n, c->q, c->inverse);
}

int cbo_ntt_cyclic_batch(uint64_t* values, uint64_t n, uint64_t batch,
                         uint64_t q, int inverse, int threads) {
    if (!values) return -1;
    ntt_ctx c = {values, n, q, inverse};
    return for_rows(batch, threads, ntt_row, &c);
}

/* ---- negacyclic composition: crypto_ntt_bench.cu:292-323, 454-528 ------- */

typedef struct {
    const uint64_t* input;
    uint64_t* output;
    uint64_t n, q, root, twist_base;
    int inverse;
} nega_ctx;

/* independent_ntt (crypto_ntt_bench.cu:454-508): O(n^2) for n <= 256, the DIT
 * loop otherwise; x n^-1 for the inverse. */
static void independent_ntt(uint64_t* values, uint64_t n, uint64_t q, uint64_t root, int inverse) {
    if (n <= 256) {
        uint64_t* out = (uint64_t*)calloc(n, sizeof(uint64_t));
        for (uint64_t k = 0; k < n; ++k) {
            uint64_t sum = 0;
            for (uint64_t j = 0; j < n; ++j) {
                const uint64_t exponent = (uint64_t)(((u128)j * k) % n);
                const uint64_t term = cbo_mod_mul(values[j] % q, cbo_mod_pow(root, exponent, q), q);
                sum += term;
                if (sum >= q) sum -= q;
            }
            out[k] = sum;
        }
        memcpy(values, out, n * sizeof(uint64_t));
        free(out);
    } else {
        dit_with_root(values, n, q, root);
    }
    if (inverse) {
        const uint64_t inverse_n = cbo_mod_pow(n, q - 2, q);
        for (uint64_t i = 0; i < n; ++i) values[i] = cbo_mod_mul(values[i], inverse_n, q);
    }
}

static int nega_row(void* context, uint64_t row) {
    nega_ctx* c = (nega_ctx*)context;
    uint64_t* slice = c->output + row * c->n;
    memcpy(slice, c->input + row * c->n, c->n * sizeof(uint64_t));
    uint64_t twist = 1;
    if (!c->inverse) {
        for (uint64_t j = 0; j < c->n; ++j) {
            slice[j] = cbo_mod_mul(slice[j], twist, c->q);
            twist = cbo_mod_mul(twist, c->twist_base, c->q);
        }
    }
    independent_ntt(slice, c->n, c->q, c->root, c->inverse);
    if (c->inverse) {
        for (uint64_t j = 0; j < c->n; ++j) {
            slice[j] = cbo_mod_mul(slice[j], twist, c->q);
            twist = cbo_mod_mul(twist, c->twist_base, c->q);
        }
    }
    return 0;
}

int cbo_ntt_negacyclic_batch(const uint64_t* input, uint64_t* output,
                             uint64_t n, uint64_t batch, uint64_t q,
                             int inverse, int threads) {
    if (!input || !output || n < 2 || !is_pow2(n) || q >= (UINT64_C(1) << 63)) return -1;
    const uint32_t log_n = log2_exact(n);
    if ((q - 1) % (2 * n) != 0) return -1;
    const uint64_t omega = cbo_find_primitive_root(log_n, q);
    if (omega == 0) return -1;
    const uint64_t psi = cbo_find_psi(log_n, q, omega);
    if (psi == 0) return -1;
    nega_ctx c;
    c.input = input;
    c.output = output;
    c.n = n;
    c.q = q;
    c.inverse = inverse;
    c.root = inverse ? cbo_mod_pow(omega, q - 2, q) : omega; /* root_for_direction :450-452 */
    c.twist_base = inverse ? cbo_mod_pow(psi, q - 2, q) : psi;
    return for_rows(batch, threads, nega_row, &c);
}

/* ---- RNS reference: tests/test_rns_ntt.cu:62-111 ------------------------ */

int cbo_rns_reference(const uint64_t* physical, uint64_t* result, uint32_t log_n,
                      uint64_t q, uint64_t root, int negacyclic, int inverse,
                      int input_bit_reversed, int output_bit_reversed) {
    if (!physical || !result || log_n == 0 || log_n > 30 || q < 3) return -1;
    const uint64_t n = UINT64_C(1) << log_n;
    uint64_t* values = (uint64_t*)malloc(n * sizeof(uint64_t));
    if (!values) return -1;
    for (uint64_t j = 0; j < n; ++j)
        values[j] = physical[input_bit_reversed ? reverse_bits(j, log_n) : j];
    if (negacyclic && !inverse) {
        uint64_t twist = 1;
        for (uint64_t j = 0; j < n; ++j) {
            values[j] = cbo_mod_mul(values[j], twist, q);
            twist = cbo_mod_mul(twist, root, q);
        }
    }
    uint64_t omega = negacyclic ? cbo_mod_mul(root, root, q) : root;
    if (inverse) omega = cbo_mod_pow(omega, q - 2, q);
    for (uint64_t j = 0; j < n; ++j) {
        const uint64_t r = reverse_bits(j, log_n);
        if (j < r) {
            const uint64_t t = values[j];
            values[j] = values[r];
            values[r] = t;
        }
    }
    for (uint64_t length = 2; length <= n; length *= 2) {
        const uint64_t step = cbo_mod_pow(omega, n / length, q);
        for (uint64_t base = 0; base < n; base += length) {
            uint64_t twiddle = 1;
            for (uint64_t j = 0; j < length / 2; ++j) {
                const uint64_t a = values[base + j];
                const uint64_t b = cbo_mod_mul(values[base + j + length / 2], twiddle, q);
                values[base + j] = (uint64_t)(((u128)a + b) % q);
                values[base + j + length / 2] = (uint64_t)(((u128)a + q - b) % q);
                twiddle = cbo_mod_mul(twiddle, step, q);
            }
        }
    }
    if (inverse) {
        uint64_t factor = cbo_mod_pow(n, q - 2, q);
        const uint64_t step = negacyclic ? cbo_mod_pow(root, q - 2, q) : 1;
        for (uint64_t j = 0; j < n; ++j) {
            values[j] = cbo_mod_mul(values[j], factor, q);
            factor = cbo_mod_mul(factor, step, q);
        }
    }
    for (uint64_t j = 0; j < n; ++j)
        result[output_bit_reversed ? reverse_bits(j, log_n) : j] = values[j];
    free(values);
    return 0;
}

typedef struct {
    const uint64_t* input;
    uint64_t* output;
    uint32_t log_n;
    const uint64_t *moduli, *roots;
    int negacyclic, inverse, in_rev, out_rev;
} rns_ctx;

static int rns_row(void* context, uint64_t p) {
    rns_ctx* c = (rns_ctx*)context;
    const uint64_t n = UINT64_C(1) << c->log_n;
    return cbo_rns_reference(c->input + p * n, c->output + p * n, c->log_n, c->moduli[p],
                             c->roots[p], c->negacyclic, c->inverse, c->in_rev, c->out_rev);
}

int cbo_rns_batch(const uint64_t* input, uint64_t* output, uint32_t log_n,
                  const uint64_t* moduli, const uint64_t* roots, uint64_t count,
                  int negacyclic, int inverse, int input_bit_reversed,
                  int output_bit_reversed, int threads) {
    if (!input || !output || !moduli || !roots) return -1;
    rns_ctx c = {input, output, log_n, moduli, roots, negacyclic, inverse,
                 input_bit_reversed, output_bit_reversed};
    return for_rows(count, threads, rns_row, &c);
}
