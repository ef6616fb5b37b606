/*
 * Restatement of the single-precision exponential used by glibc 2.35 on
 * x86_64 (sysdeps/ieee754/flt-32/e_expf.c, the algorithm published in Arm
 * Optimized Routines by Szabolcs Nagy, 2017; glibc's x86_64 build selects the
 * FMA variant on CPUs with FMA). TEST INFRASTRUCTURE ONLY: it is the checker
 * that pins the GPU engine's `expf` restatement (lumen_amd/csrc) to the
 * system libm that the Rust reference calls (`f32::exp` -> `expf`).
 *
 * Algorithm (published method): x*N/ln2 = k + r with N = 32, |r| <= 1/2,
 * k rounded to nearest via the 1.5*2^52 shift trick; 2^(k/N) is built from a
 * 32-entry table of 2^(i/N) in double with k's high part added to the
 * exponent; 2^(r/N) ~ 1 + C2 r + C1 r^2 + C0 r^3 evaluated in double and the
 * product rounded once to float. Special cases: |x| >= 88 handles -inf -> 0,
 * inf/NaN -> x + x, overflow above log(2^128) and underflow below
 * log(2^-150).
 *
 * The table is not stored: entry i is the double nearest 2^(i/32) (computed
 * here in long double), minus i << 47 so that adding k << 47 restores the
 * exponent of 2^(k/32).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static uint64_t g_tab[32];
static int g_init;

static inline double asd(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static inline uint64_t asu64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline uint32_t asu(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

void ref_expf_table(uint64_t out[32]) {
    for (int i = 0; i < 32; i++) {
        long double v = exp2l((long double)i / 32.0L);
        out[i] = asu64((double)v) - ((uint64_t)i << 47);
    }
}

float ref_glibc_expf(float x) {
    static const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    static const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    static const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
    static const double SHIFT = 0x1.8p+52;
    static const double INVLN2N = 0x1.71547652b82fep+0 * 32;
    if (!g_init) { ref_expf_table(g_tab); g_init = 1; }
    uint32_t abstop = (asu(x) >> 20) & 0x7ff;
    if (abstop >= (asu(88.0f) >> 20)) {
        if (asu(x) == asu(-INFINITY)) return 0.0f;
        if (abstop >= (asu(INFINITY) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double kd = fma(INVLN2N, xd, SHIFT);
    uint64_t ki = asu64(kd);
    kd -= SHIFT;
    double r = fma(INVLN2N, xd, -kd);
    uint64_t t = g_tab[ki % 32] + (ki << 47);
    double s = asd(t);
    double z = fma(C0, r, C1);
    double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(z, r2, y);
    y = y * s;
    return (float)y;
}

/* Compares the restatement with the system expf over `count` consecutive
 * bit patterns starting at `start` (NaN patterns skipped). Returns the
 * number of mismatching results and stores the first mismatch's input. */
uint64_t ref_expf_check_range(uint32_t start, uint64_t count, uint32_t *first_bad) {
    uint64_t bad = 0;
    for (uint64_t i = 0; i < count; i++) {
        uint32_t u = (uint32_t)(start + i);
        float x;
        memcpy(&x, &u, 4);
        if (isnan(x)) continue;
        float a = ref_glibc_expf(x);
        float b = expf(x);
        if (asu(a) != asu(b)) {
            if (!bad && first_bad) *first_bad = u;
            bad++;
        }
    }
    return bad;
}
