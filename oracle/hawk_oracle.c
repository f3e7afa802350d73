/* hawk_oracle.c — TEST INFRASTRUCTURE, not product code.
 *
 * A plain-C restatement of what hawk's HOST target computes for the five
 * benchmark kernels, used only as the parity checker (tests/, the smoke
 * check of __graft_entry__.py) and as the CPU baseline of bench.py.  Nothing
 * in hawk_amd/ links, loads or calls it.
 *
 * It is built the way hawk builds a host .so in its exact `native` profile
 * (reference hawk/compile/toolchain.py:956-987): gcc -O3 -march=native
 * -mprefer-vector-width=512 -ffp-contract=off -fno-math-errno, so every
 * operation below is one IEEE operation and the transcendentals are glibc's
 * (reference tests/test_math_parity.py:279: host `native` == glibc bit for bit).
 * The per-sample loops have the host wrapper's shape: a serial loop over
 * [base, base+count) (reference hawk/emit/host.py:213-217, :1450-1460).
 *
 * Planes are component-major [component][sample] (reference
 * hawk/emit/wrapper.py:1029-1055): component c of sample s at c*n + s.
 *
 * How each function is pinned (golden vectors, closed forms, brute force,
 * finite differences, invariants) is tested in tests/test_oracle.py; every
 * function here has at least one such check.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HKO_EXPORT __attribute__((visibility("default")))

/* ---- config 1: scale(x, a, b) = a*x + b ------------------------------------
 * The kernel `return a * x + b` (reference README.md:44-56): mul then add. */
HKO_EXPORT void hko_scale(const double* x, double a, double b, double* out,
                          int64_t base, int64_t count) {
#pragma GCC ivdep
    for (int64_t i = base; i < base + count; ++i) out[i] = (a * x[i]) + b;
}

/* ---- config 2: energy = 0.5 * dot(v, v), its VJP and its JVP ---------------
 * dot adds its products left to right.  VJP by reference hawk/diff/rules.py:
 * mul(0.5, d) sends g*0.5 to d, and dot sends (g*0.5)*v to each of its two
 * operands, accumulated held + new.  JVP: 0.5 * (dot(dv, v) + dot(v, dv)). */
HKO_EXPORT void hko_energy(const double* v, int64_t n, double* out, int64_t base, int64_t count) {
#pragma GCC ivdep
    for (int64_t i = base; i < base + count; ++i) {
        const double a = v[i], b = v[n + i], c = v[2 * n + i];
        out[i] = 0.5 * (((a * a) + (b * b)) + (c * c));
    }
}

HKO_EXPORT void hko_energy_vjp(const double* v, const double* bar_out, int64_t n, double* bar_v,
                               int64_t base, int64_t count) {
#pragma GCC ivdep
    for (int64_t i = base; i < base + count; ++i) {
        const double g = bar_out[i] * 0.5;
        for (int c = 0; c < 3; ++c) {
            const double t = g * v[c * n + i];
            bar_v[c * n + i] = t + t;
        }
    }
}

HKO_EXPORT void hko_energy_jvp(const double* v, const double* dv, int64_t n, double* dot_out,
                               int64_t base, int64_t count) {
#pragma GCC ivdep
    for (int64_t i = base; i < base + count; ++i) {
        const double a = v[i], b = v[n + i], c = v[2 * n + i];
        const double da = dv[i], db = dv[n + i], dc = dv[2 * n + i];
        const double d1 = ((da * a) + (db * b)) + (dc * c);
        const double d2 = ((a * da) + (b * db)) + (c * dc);
        dot_out[i] = 0.5 * (d1 + d2);
    }
}

/* ---- config 5a: the 8-stage chain --------------------------------------- */
static inline double chain1(double x) {
    const double t1 = exp(x);
    const double t2 = sin(t1);
    const double t3 = (1.5 * t2) + 0.25;
    const double t4 = tanh(t3);
    const double t5 = sqrt(fabs(t4) + 1.0);
    const double t6 = (t5 * t5) - x;
    const double t7 = exp(-fabs(t6));
    return (t7 * x) + t4;
}

HKO_EXPORT void hko_chain(const double* x, double* y, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) y[i] = chain1(x[i]);
}

/* dy/dx of the chain, by the chain rule written out stage by stage (not by
 * the derivative transform under test; pinned by central differences of
 * chain1).  d|u|/du is +1 at u >= 0 and -1 below, as reference
 * hawk/diff/rules.py's abs rule takes it. */
static inline double chain1_dx(double x) {
    const double t1 = exp(x), d1 = t1;
    const double t2 = sin(t1), d2 = cos(t1) * d1;
    const double t3 = (1.5 * t2) + 0.25, d3 = 1.5 * d2;
    const double t4 = tanh(t3), d4 = (1.0 - t4 * t4) * d3;
    const double t5 = sqrt(fabs(t4) + 1.0), d5 = (0.5 / t5) * (t4 >= 0.0 ? d4 : -d4);
    const double t6 = (t5 * t5) - x, d6 = 2.0 * t5 * d5 - 1.0;
    const double t7 = exp(-fabs(t6)), d7 = -t7 * (t6 >= 0.0 ? d6 : -d6);
    return (d7 * x + t7) + d4;
}

/* The chain's derivatives through its three sinks (y per sample, the total,
 * the bins at key): the VJP bar_x = dy/dx * (bar_y + bar_total + bar_bins[key])
 * (a key outside [0, cells) reads 0: the scatter's skip key), and the JVP's
 * per-sample tangent dot_y = dy/dx * dot_x (its total and bins are the ordered
 * sum and scatter of dot_y). */
HKO_EXPORT void hko_chain_vjp(const double* x, const int32_t* key, const double* bar_y, double bar_total,
                              const double* bar_bins, int64_t cells, int64_t n, double* bar_x) {
    for (int64_t i = 0; i < n; ++i) {
        const int64_t k = key[i];
        const double g = (bar_y[i] + bar_total) + ((k >= 0 && k < cells) ? bar_bins[k] : 0.0);
        bar_x[i] = chain1_dx(x[i]) * g;
    }
}

HKO_EXPORT void hko_chain_jvp(const double* x, const double* dot_x, int64_t n, double* dot_y) {
    for (int64_t i = 0; i < n; ++i) dot_y[i] = chain1_dx(x[i]) * dot_x[i];
}

/* The transcendentals one at a time (for ULP tests of the device's). */
HKO_EXPORT void hko_libm(int which, const double* x, double* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        switch (which) {
            case 0: y[i] = exp(x[i]); break;
            case 1: y[i] = sin(x[i]); break;
            case 2: y[i] = tanh(x[i]); break;
            case 3: y[i] = sqrt(x[i]); break;
            case 4: y[i] = cos(x[i]); break;
            default: y[i] = log(x[i]); break;
        }
    }
}

/* ---- config 5b: the fixed-tree ordered sum --------------------------------
 * Reference hawk/emit/team.py:208-278 (`_block_part`, host form) and
 * :173-192 (`_block`, gp form): group g's 1024 lanes accumulate rows
 * b + t (b = g*1024, g*1024 + 65536, ...) into sh[t] from 0; the halving tree
 * sh[i] += sh[i+w], w = 512..1, gives gp[g]; the same tree, w = 32..1, over
 * the 64 gp values gives the sum. */
#define HKO_V 65536
#define HKO_W 1024
#define HKO_G 64

static double group_part(const double* u, int64_t rows, int g) {
    double sh[HKO_W];
    for (int t = 0; t < HKO_W; ++t) sh[t] = 0.0;
    for (int64_t b = (int64_t)g * HKO_W; b < rows; b += HKO_V) {
        const int64_t m = rows - b < HKO_W ? rows - b : HKO_W;
        for (int64_t t = 0; t < m; ++t) sh[t] += u[b + t];
    }
    for (int w = HKO_W / 2; w > 0; w >>= 1)
        for (int i = 0; i < w; ++i) sh[i] += sh[i + w];
    return sh[0];
}

static double fold_groups(double* gp) {
    for (int w = HKO_G / 2; w > 0; w >>= 1)
        for (int i = 0; i < w; ++i) gp[i] += gp[i + w];
    return gp[0];
}

/* ---- default-policy sample sum: compensated rows, canonical finish -------
 * Reference hawk/emit/wrapper.py:542-665 (sampleSumRow_: a row of 32 slots,
 * slot l combined with slot l + off for off = 16, 8, 4, 2, 1 by pairCombine_)
 * and hawk/_cells.py:44-119 (twoSumErr, Neumaier add, pair combine, leaves of
 * 256 slots x 16 rows, the in-leaf halving tree, pairwise levels, hi + comp). */
static int fin(double x) { return (x - x) == 0.0; }

static double two_sum_err(double a, double b, double s) {
    const int big_a = fabs(a) >= fabs(b);
    const double big = big_a ? a : b, small = big_a ? b : a;
    return fin(s) ? (small - (s - big)) + 0.0 : NAN;
}

static void pair_add(double* h, double* c, double h2, double c2) {
    const double s = *h + h2;
    *c = fin(s) ? (*c + c2) + two_sum_err(*h, h2, s) : 0.0;
    *h = s;
}

static void neumaier_add(double* h, double* c, double x, double xc) {
    const double s = *h + x;
    *c = fin(s) ? *c + two_sum_err(*h, x, s) : 0.0;
    *c = fin(s) ? *c + xc : 0.0;
    *h = s;
}

/* Rows of 32 terms (a ragged last row padded with +0). */
HKO_EXPORT void hko_row_sums(const double* t, int64_t n, double* hi, double* comp) {
    const int64_t rows = (n + 31) / 32;
    for (int64_t r = 0; r < rows; ++r) {
        double h[32], c[32];
        for (int l = 0; l < 32; ++l) {
            h[l] = r * 32 + l < n ? t[r * 32 + l] : 0.0;
            c[l] = 0.0;
        }
        for (int off = 16; off >= 1; off >>= 1)
            for (int l = 0; l < off; ++l) pair_add(&h[l], &c[l], h[l + off], c[l + off]);
        hi[r] = h[0];
        comp[r] = c[0];
    }
}

/* The leaf of rows [0, cnt) of (hi, comp), cnt <= 4096. */
static void rows_leaf(const double* hi, const double* comp, int cnt, double* lh, double* lc) {
    double sh[256], sc[256];
    const int live = cnt < 256 ? cnt : 256;
    for (int s = 0; s < live; ++s) {
        sh[s] = hi[s];
        sc[s] = fin(hi[s]) ? comp[s] : 0.0;
    }
    for (int k = 1; k < 16; ++k) {
        const int m = live < cnt - k * 256 ? live : cnt - k * 256;
        if (m <= 0) break;
        for (int s = 0; s < m; ++s) neumaier_add(&sh[s], &sc[s], hi[k * 256 + s], comp[k * 256 + s]);
    }
    for (int off = 128; off > 0; off >>= 1) {
        const int lim = live > off ? (off < live - off ? off : live - off) : 0;
        for (int s = 0; s < lim; ++s) pair_add(&sh[s], &sc[s], sh[s + off], sc[s + off]);
    }
    *lh = sh[0];
    *lc = sc[0];
}

HKO_EXPORT double hko_rows_finish(const double* hi, const double* comp, int64_t rows) {
    if (rows <= 0) return 0.0;
    const int64_t leaves = (rows + 4095) / 4096;
    double* vh = (double*)malloc(sizeof(double) * (size_t)leaves);
    double* vc = (double*)malloc(sizeof(double) * (size_t)leaves);
    for (int64_t j = 0; j < leaves; ++j) {
        const int64_t rest = rows - j * 4096;
        rows_leaf(hi + j * 4096, comp + j * 4096, (int)(rest < 4096 ? rest : 4096), &vh[j], &vc[j]);
    }
    int64_t m = leaves;
    while (m > 1) {
        const int64_t pairs = m / 2;
        for (int64_t p = 0; p < pairs; ++p) {
            double h = vh[2 * p], c = vc[2 * p];
            pair_add(&h, &c, vh[2 * p + 1], vc[2 * p + 1]);
            vh[p] = h;
            vc[p] = c;
        }
        if (m & 1) {
            vh[pairs] = vh[m - 1];
            vc[pairs] = vc[m - 1];
        }
        m = pairs + (m & 1);
    }
    const double out = fin(vh[0]) ? vh[0] + vc[0] : vh[0];
    free(vh);
    free(vc);
    return out;
}

/* The float32 scalar mode's default-policy sum: the same rows and finish in
 * float32 arithmetic (the reference's rows are the stage's `Real`, float in
 * that mode, and hawk/_cells.py:44-119 runs the finish in the rows' dtype). */
static int fin_f(float x) { return (x - x) == 0.0f; }

static float two_sum_err_f(float a, float b, float s) {
    const int big_a = fabsf(a) >= fabsf(b);
    const float big = big_a ? a : b, small = big_a ? b : a;
    return fin_f(s) ? (small - (s - big)) + 0.0f : NAN;
}

static void pair_add_f(float* h, float* c, float h2, float c2) {
    const float s = *h + h2;
    *c = fin_f(s) ? (*c + c2) + two_sum_err_f(*h, h2, s) : 0.0f;
    *h = s;
}

static void neumaier_add_f(float* h, float* c, float x, float xc) {
    const float s = *h + x;
    *c = fin_f(s) ? *c + two_sum_err_f(*h, x, s) : 0.0f;
    *c = fin_f(s) ? *c + xc : 0.0f;
    *h = s;
}

HKO_EXPORT void hko_row_sums_f32(const float* t, int64_t n, float* hi, float* comp) {
    const int64_t rows = (n + 31) / 32;
    for (int64_t r = 0; r < rows; ++r) {
        float h[32], c[32];
        for (int l = 0; l < 32; ++l) {
            h[l] = r * 32 + l < n ? t[r * 32 + l] : 0.0f;
            c[l] = 0.0f;
        }
        for (int off = 16; off >= 1; off >>= 1)
            for (int l = 0; l < off; ++l) pair_add_f(&h[l], &c[l], h[l + off], c[l + off]);
        hi[r] = h[0];
        comp[r] = c[0];
    }
}

static void rows_leaf_f(const float* hi, const float* comp, int cnt, float* lh, float* lc) {
    float sh[256], sc[256];
    const int live = cnt < 256 ? cnt : 256;
    for (int s = 0; s < live; ++s) {
        sh[s] = hi[s];
        sc[s] = fin_f(hi[s]) ? comp[s] : 0.0f;
    }
    for (int k = 1; k < 16; ++k) {
        const int m = live < cnt - k * 256 ? live : cnt - k * 256;
        if (m <= 0) break;
        for (int s = 0; s < m; ++s) neumaier_add_f(&sh[s], &sc[s], hi[k * 256 + s], comp[k * 256 + s]);
    }
    for (int off = 128; off > 0; off >>= 1) {
        const int lim = live > off ? (off < live - off ? off : live - off) : 0;
        for (int s = 0; s < lim; ++s) pair_add_f(&sh[s], &sc[s], sh[s + off], sc[s + off]);
    }
    *lh = sh[0];
    *lc = sc[0];
}

HKO_EXPORT float hko_rows_finish_f32(const float* hi, const float* comp, int64_t rows) {
    if (rows <= 0) return 0.0f;
    const int64_t leaves = (rows + 4095) / 4096;
    float* vh = (float*)malloc(sizeof(float) * (size_t)leaves);
    float* vc = (float*)malloc(sizeof(float) * (size_t)leaves);
    for (int64_t j = 0; j < leaves; ++j) {
        const int64_t rest = rows - j * 4096;
        rows_leaf_f(hi + j * 4096, comp + j * 4096, (int)(rest < 4096 ? rest : 4096), &vh[j], &vc[j]);
    }
    int64_t m = leaves;
    while (m > 1) {
        const int64_t pairs = m / 2;
        for (int64_t p = 0; p < pairs; ++p) {
            float h = vh[2 * p], c = vc[2 * p];
            pair_add_f(&h, &c, vh[2 * p + 1], vc[2 * p + 1]);
            vh[p] = h;
            vc[p] = c;
        }
        if (m & 1) {
            vh[pairs] = vh[m - 1];
            vc[pairs] = vc[m - 1];
        }
        m = pairs + (m & 1);
    }
    const float out = fin_f(vh[0]) ? vh[0] + vc[0] : vh[0];
    free(vh);
    free(vc);
    return out;
}

HKO_EXPORT float hko_sample_sum_f32(const float* t, int64_t n) {
    const int64_t rows = (n + 31) / 32;
    if (rows == 0) return 0.0f;
    float* hi = (float*)malloc(sizeof(float) * (size_t)rows);
    float* comp = (float*)malloc(sizeof(float) * (size_t)rows);
    hko_row_sums_f32(t, n, hi, comp);
    const float out = hko_rows_finish_f32(hi, comp, rows);
    free(hi);
    free(comp);
    return out;
}

HKO_EXPORT double hko_sample_sum(const double* t, int64_t n) {
    const int64_t rows = (n + 31) / 32;
    if (rows == 0) return 0.0;
    double* hi = (double*)malloc(sizeof(double) * (size_t)rows);
    double* comp = (double*)malloc(sizeof(double) * (size_t)rows);
    hko_row_sums(t, n, hi, comp);
    const double out = hko_rows_finish(hi, comp, rows);
    free(hi);
    free(comp);
    return out;
}

/* The default-policy keyed sum: each key's run of `group` values as a sample
 * sum of its own (the device's fixed order; the reference's atomic commits,
 * hawk/emit/wrapper.py:380-415, give these bits when a key spans at most two
 * warps' partials and one of its possible results otherwise). */
HKO_EXPORT void hko_keyed_sample_sum(const double* u, int64_t n, int64_t group, double* out) {
    for (int64_t k = 0; k * group < n; ++k) out[k] = hko_sample_sum(u + k * group, group);
}

/* ---- hawk.max / hawk.min: row extremes, the canonical finish -------------
 * Reference hawk/emit/wrapper.py:543-600 (ssExtreme_: the extreme of two
 * values that ignores a NaN operand; ssIdentity_: -inf (max) / +inf (min)
 * past the last sample; sampleSumRow_: slot l with slot l + off, off = 16 ..
 * 1) and hawk/_cells.py:66-71 with `finish` (the sum's leaves and levels,
 * every add np.where(a > b, a, b) for max, np.where(a < b, a, b) for min, so
 * a NaN partial on the left gives way and one on the right wins).
 * op 1 = max, 2 = min; T is double or float. */
#define HKO_EXTREME_FNS(T, SUF)                                                          \
static T ss_extreme##SUF(int op, T a, T b) {                                             \
    if (a != a) return b;                                                                \
    if (b != b) return a;                                                                \
    return op == 1 ? (b > a ? b : a) : (b < a ? b : a);                                  \
}                                                                                        \
static T tree_extreme##SUF(int op, T a, T b) { return op == 1 ? (a > b ? a : b) : (a < b ? a : b); } \
HKO_EXPORT void hko_row_extremes##SUF(const T* t, int64_t n, int op, T* hi) {            \
    const int64_t rows = (n + 31) / 32;                                                  \
    const T ident = op == 1 ? -(T)INFINITY : (T)INFINITY;                                \
    for (int64_t r = 0; r < rows; ++r) {                                                 \
        T h[32];                                                                         \
        for (int l = 0; l < 32; ++l) h[l] = r * 32 + l < n ? t[r * 32 + l] : ident;      \
        for (int off = 16; off >= 1; off >>= 1)                                          \
            for (int l = 0; l < off; ++l) h[l] = ss_extreme##SUF(op, h[l], h[l + off]);  \
        hi[r] = h[0];                                                                    \
    }                                                                                    \
}                                                                                        \
HKO_EXPORT T hko_rows_extreme##SUF(const T* hi, int64_t rows, int op) {                  \
    if (rows <= 0) return op == 1 ? -(T)INFINITY : (T)INFINITY;                          \
    const int64_t leaves = (rows + 4095) / 4096;                                         \
    T* vh = (T*)malloc(sizeof(T) * (size_t)leaves);                                      \
    for (int64_t j = 0; j < leaves; ++j) {                                               \
        const T* x = hi + j * 4096;                                                      \
        const int64_t rest = rows - j * 4096;                                            \
        const int cnt = (int)(rest < 4096 ? rest : 4096), live = cnt < 256 ? cnt : 256;  \
        T sh[256];                                                                       \
        for (int s = 0; s < live; ++s) sh[s] = x[s];                                     \
        for (int k = 1; k < 16; ++k) {                                                   \
            const int m = live < cnt - k * 256 ? live : cnt - k * 256;                   \
            if (m <= 0) break;                                                           \
            for (int s = 0; s < m; ++s) sh[s] = tree_extreme##SUF(op, sh[s], x[k * 256 + s]); \
        }                                                                                \
        for (int off = 128; off > 0; off >>= 1) {                                        \
            const int lim = live > off ? (off < live - off ? off : live - off) : 0;      \
            for (int s = 0; s < lim; ++s) sh[s] = tree_extreme##SUF(op, sh[s], sh[s + off]); \
        }                                                                                \
        vh[j] = sh[0];                                                                   \
    }                                                                                    \
    int64_t m = leaves;                                                                  \
    while (m > 1) {                                                                      \
        const int64_t pairs = m / 2;                                                     \
        for (int64_t q = 0; q < pairs; ++q) vh[q] = tree_extreme##SUF(op, vh[2 * q], vh[2 * q + 1]); \
        if (m & 1) vh[pairs] = vh[m - 1];                                                \
        m = pairs + (m & 1);                                                             \
    }                                                                                    \
    const T out = vh[0];                                                                 \
    free(vh);                                                                            \
    return out;                                                                          \
}                                                                                        \
HKO_EXPORT T hko_sample_extreme##SUF(const T* t, int64_t n, int op) {                    \
    const int64_t rows = (n + 31) / 32;                                                  \
    if (rows == 0) return op == 1 ? -(T)INFINITY : (T)INFINITY;                          \
    T* hi = (T*)malloc(sizeof(T) * (size_t)rows);                                        \
    hko_row_extremes##SUF(t, n, op, hi);                                                 \
    const T out = hko_rows_extreme##SUF(hi, rows, op);                                   \
    free(hi);                                                                            \
    return out;                                                                          \
}

HKO_EXTREME_FNS(double, )
HKO_EXTREME_FNS(float, _f32)

/* ---- banded reductions: double-double band accumulators ----------------
 * The banded scalar mode's reductions (reference hawk/emit/wrapper.py:140
 * `BANDED`, hawk/emit/team.py:26-49 and :225-245: every partial is a
 * compensated band accumulator, folded in the float64 stages' fixed order,
 * one value stored at the end).  Here a band is a normalised double-double
 * (h, l), |l| <= ulp(h)/2, with the additions of Hida, Li and Bailey's QD
 * library (TwoSum, quick-two-sum; the "accurate" double-double add); a
 * non-finite leading sum drops the low part.  The stored cell is h. */
typedef struct { double h, l; } hko_band;

static hko_band band_two(double a, double b) {          /* TwoSum: s + e == a + b exactly */
    const double s = a + b, bb = s - a;
    const hko_band r = {s, (a - (s - bb)) + (b - bb)};
    return r;
}

static hko_band band_quick(double a, double b) {        /* quick-two-sum, |a| >= |b| (or a == 0) */
    const double s = a + b;
    const hko_band r = {s, b - (s - a)};
    return r;
}

/* A virtual lane's run of rows (the banded ordered sum): Neumaier's
 * compensated sum, the running sum s one addition a row and each addition's
 * exact error added to c beside it (the larger operand first), renormalised
 * into a band once, at the run's end, by TwoSum of (s, c); a non-finite s
 * drops c.  (The reference's accumulator likewise renormalises only every
 * BandAccum::period terms, hawk/emit/team.py:32-34.) */
typedef struct { double s, c; } hko_lane;

static void lane_add(hko_lane* a, double x) {
    const double t = a->s + x;
    const double e = fabs(a->s) >= fabs(x) ? (a->s - t) + x : (x - t) + a->s;
    a->c = a->c + e;
    a->s = t;
}

static hko_band lane_band(hko_lane a) {
    if (!fin(a.s)) { const hko_band r = {a.s, 0.0}; return r; }
    return band_two(a.s, a.c);
}

static hko_band band_add(hko_band a, hko_band b) {
    hko_band s = band_two(a.h, b.h);
    if (!fin(s.h)) { s.l = 0.0; return s; }
    const hko_band t = band_two(a.l, b.l);
    s = band_quick(s.h, s.l + t.h);
    return band_quick(s.h, s.l + t.l);
}

/* Rows of 32 terms, each term the band (t, +0), combined by the pairs (l, l ^ 16), ..., (l, l ^ 1)
 * of the default sum's row (the band add is symmetric, so every lane of the row ends with these bits). */
HKO_EXPORT void hko_band_row_sums(const double* t, int64_t n, double* hi, double* lo) {
    const int64_t rows = (n + 31) / 32;
    for (int64_t r = 0; r < rows; ++r) {
        hko_band v[32];
        for (int l = 0; l < 32; ++l) {
            v[l].h = r * 32 + l < n ? t[r * 32 + l] : 0.0;
            v[l].l = 0.0;
        }
        for (int off = 16; off >= 1; off >>= 1)
            for (int l = 0; l < off; ++l) v[l] = band_add(v[l], v[l + off]);
        hi[r] = v[0].h;
        lo[r] = v[0].l;
    }
}

/* The canonical finish of the default sum (leaves of 256 slots x 16 rows, the in-leaf halving tree,
 * pairwise levels over the leaves), every add a band add; the cell is the final band's h. */
static hko_band band_leaf(const double* hi, const double* lo, int cnt) {
    hko_band sh[256];
    const int live = cnt < 256 ? cnt : 256;
    for (int s = 0; s < live; ++s) {
        sh[s].h = hi[s];
        sh[s].l = lo[s];
    }
    for (int k = 1; k < 16; ++k) {
        const int m = live < cnt - k * 256 ? live : cnt - k * 256;
        if (m <= 0) break;
        for (int s = 0; s < m; ++s) {
            const hko_band row = {hi[k * 256 + s], lo[k * 256 + s]};
            sh[s] = band_add(sh[s], row);
        }
    }
    for (int off = 128; off > 0; off >>= 1) {
        const int lim = live > off ? (off < live - off ? off : live - off) : 0;
        for (int s = 0; s < lim; ++s) sh[s] = band_add(sh[s], sh[s + off]);
    }
    return sh[0];
}

HKO_EXPORT double hko_band_rows_finish(const double* hi, const double* lo, int64_t rows) {
    if (rows <= 0) return 0.0;
    const int64_t leaves = (rows + 4095) / 4096;
    hko_band* v = (hko_band*)malloc(sizeof(hko_band) * (size_t)leaves);
    for (int64_t j = 0; j < leaves; ++j) {
        const int64_t rest = rows - j * 4096;
        v[j] = band_leaf(hi + j * 4096, lo + j * 4096, (int)(rest < 4096 ? rest : 4096));
    }
    int64_t m = leaves;
    while (m > 1) {
        const int64_t pairs = m / 2;
        for (int64_t p = 0; p < pairs; ++p) v[p] = band_add(v[2 * p], v[2 * p + 1]);
        if (m & 1) v[pairs] = v[m - 1];
        m = pairs + (m & 1);
    }
    const double out = v[0].h;
    free(v);
    return out;
}

HKO_EXPORT double hko_band_sample_sum(const double* t, int64_t n) {
    const int64_t rows = (n + 31) / 32;
    if (rows == 0) return 0.0;
    double* hi = (double*)malloc(sizeof(double) * (size_t)rows);
    double* lo = (double*)malloc(sizeof(double) * (size_t)rows);
    hko_band_row_sums(t, n, hi, lo);
    const double out = hko_band_rows_finish(hi, lo, rows);
    free(hi);
    free(lo);
    return out;
}

/* The banded ordered sum, reference hawk/emit/team.py:26-30 (BAND_LANES = 128, BAND_VIRTUAL_LANES =
 * 128 x 64) and :225-245 (the `cells` form of `_block_part`): group g's 128 virtual lanes l = g*128 + t
 * each add rows l, l + 8192, ... in order into one lane accumulator from (+0, +0), the halving tree
 * w = 64..1 over the group's 128 bands gives gp[g], and the tree w = 32..1 over the 64 group bands
 * (:160-171) gives the sum; the cell is the final band's h. */
#define HKO_BW 128
#define HKO_BV (HKO_BW * HKO_G)
static hko_band band_group_part(const double* u, int64_t rows, int g) {
    hko_band sh[HKO_BW];
    for (int t = 0; t < HKO_BW; ++t) {
        hko_lane a = {0.0, 0.0};
        for (int64_t r = (int64_t)g * HKO_BW + t; r < rows; r += HKO_BV) lane_add(&a, u[r]);
        sh[t] = lane_band(a);
    }
    for (int w = HKO_BW / 2; w > 0; w >>= 1)
        for (int i = 0; i < w; ++i) sh[i] = band_add(sh[i], sh[i + w]);
    return sh[0];
}

HKO_EXPORT double hko_band_ordered_sum(const double* u, int64_t n) {
    hko_band gp[HKO_G];
    for (int g = 0; g < HKO_G; ++g) gp[g] = band_group_part(u, n, g);
    for (int w = HKO_G / 2; w > 0; w >>= 1)
        for (int i = 0; i < w; ++i) gp[i] = band_add(gp[i], gp[i + w]);
    return gp[0].h;
}

HKO_EXPORT double hko_ordered_sum(const double* u, int64_t n) {
    double gp[HKO_G];
    for (int g = 0; g < HKO_G; ++g) gp[g] = group_part(u, n, g);
    return fold_groups(gp);
}

/* The ordered sum in the float32 mode: the reference's team stages are
 * written over `Real` (hawk/emit/team.py:248-261), so in float32 every lane
 * sum and every tree level is a float addition. */
static float group_part_f(const float* u, int64_t rows, int g) {
    float sh[HKO_W];
    for (int t = 0; t < HKO_W; ++t) sh[t] = 0.0f;
    for (int64_t b = (int64_t)g * HKO_W; b < rows; b += HKO_V) {
        const int64_t m = rows - b < HKO_W ? rows - b : HKO_W;
        for (int64_t t = 0; t < m; ++t) sh[t] += u[b + t];
    }
    for (int w = HKO_W / 2; w > 0; w >>= 1)
        for (int i = 0; i < w; ++i) sh[i] += sh[i + w];
    return sh[0];
}

HKO_EXPORT float hko_ordered_sum_f32(const float* u, int64_t n) {
    float gp[HKO_G];
    for (int g = 0; g < HKO_G; ++g) gp[g] = group_part_f(u, n, g);
    for (int w = HKO_G / 2; w > 0; w >>= 1)
        for (int i = 0; i < w; ++i) gp[i] += gp[i + w];
    return gp[0];
}

HKO_EXPORT void hko_keyed_ordered_sum_f32(const float* u, int64_t n, int64_t group, float* out) {
    for (int64_t k = 0; k * group < n; ++k) out[k] = hko_ordered_sum_f32(u + k * group, group);
}

/* hawk.sum(x, over=<trailing lane axes>, policy="ordered"): key k's rows are
 * u[k*group .. (k+1)*group), each key takes the ordered sum's tree on its own
 * rows (reference hawk/emit/team.py:115-205 and :208-278: block b is group
 * b % 64 of key b / 64; the gp stage folds a key's 64 group values). */
HKO_EXPORT void hko_keyed_ordered_sum(const double* u, int64_t n, int64_t group, double* out) {
    for (int64_t k = 0; k * group < n; ++k) out[k] = hko_ordered_sum(u + k * group, group);
}

/* The ordered gradient's log fold (reference hawk/diff/ordered.py,
 * hawk/ir/team.py:684-693, hawk/emit/team.py:281-312 `_fold`): for key k and
 * slot e, the key's rows contributions values[e*stride + k*rows + r] are
 * added in lane order from +0 and STORED into out[cells_log[e*keys + k]].
 * Pairs run in (slot, key) order, so of two pairs naming one cell the later
 * one's sum is what remains (the device reports such a cell instead).
 * Returns 1 when a cell is outside [0, cells) (not stored), else 0. */
HKO_EXPORT int hko_keyed_log_fold(const double* values, int64_t stride, const int32_t* cells_log, int64_t keys,
                                  int64_t rows, int32_t width, double* out, int64_t cells) {
    int bad = 0;
    for (int32_t e = 0; e < width; ++e) {
        for (int64_t k = 0; k < keys; ++k) {
            const double* p = values + (int64_t)e * stride + k * rows;
            double s = 0.0;
            for (int64_t r = 0; r < rows; ++r) s += p[r];
            const int32_t c = cells_log[(int64_t)e * keys + k];
            if (c < 0 || c >= cells) bad = 1;
            else out[c] = s;
        }
    }
    return bad;
}

/* The same fold in the float32 mode: each key's run added in float from +0. */
HKO_EXPORT int hko_keyed_log_fold_f32(const float* values, int64_t stride, const int32_t* cells_log, int64_t keys,
                                      int64_t rows, int32_t width, float* out, int64_t cells) {
    int bad = 0;
    for (int32_t e = 0; e < width; ++e) {
        for (int64_t k = 0; k < keys; ++k) {
            const float* p = values + (int64_t)e * stride + k * rows;
            float s = 0.0f;
            for (int64_t r = 0; r < rows; ++r) s += p[r];
            const int32_t c = cells_log[(int64_t)e * keys + k];
            if (c < 0 || c >= cells) bad = 1;
            else out[c] = s;
        }
    }
    return bad;
}

/* ---- hawk.chain: four members passing values by name ----------------------
 * Reference hawk/trace/chain.py (and its tests/test_chain.py fixture): a =
 * (sin x, cos x, x*0.5); b = exp(-((a0*a0 + a1*a1) + a2*a2)) + x;
 * acc = acc + b*b; y = a * b.  The chain runs them as one kernel; so does
 * this loop (a and b stay local). */
HKO_EXPORT void hko_chain_members(const double* x, double* acc, double* y, int64_t n, int64_t base,
                                  int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        const double xi = x[i];
        const double a0 = sin(xi), a1 = cos(xi), a2 = xi * 0.5;
        const double b = exp(-((a0 * a0 + a1 * a1) + a2 * a2)) + xi;
        acc[i] = acc[i] + b * b;
        y[i] = a0 * b;
        y[n + i] = a1 * b;
        y[2 * n + i] = a2 * b;
    }
}

/* ---- the net axis: many small models in one launch ------------------------
 * Reference tests/test_net_axis.py (its kernel file _net_axis_kernels.py):
 * lanes are (net, sample), s samples per net; net k's weights
 * w[k*24 + 3h .. 3h+2] = (a_h, b_h, c_h) of unit h < 8, and mask[k*8 + h]
 * switches unit h off.  A sample's term is r*r, r = pred - y, pred =
 * sum over h, in order from 0*x, of (mask_h * c_h) * tanh(a_h*x + b_h).  Net
 * k's loss is the ordered sum of its s terms (the keyed ordered sum: each
 * key's run takes the fixed tree); its gradient wrt w adds each weight's
 * per-sample contributions bar_out[k] * d(term)/dw in lane order from +0
 * (the ordered fold's order). */
static double net_residual(const double* w, const double* m, double x, double y, double* t) {
    double pred = 0.0 * x;
    for (int h = 0; h < 8; ++h) {
        t[h] = tanh(w[3 * h] * x + w[3 * h + 1]);
        pred = pred + m[h] * w[3 * h + 2] * t[h];
    }
    return pred - y;
}

HKO_EXPORT void hko_net_loss(const double* w, const double* mask, const double* x, const double* y, int64_t s,
                             double* out, int64_t k0, int64_t k1) {
    double* terms = (double*)malloc(sizeof(double) * (size_t)(s > 0 ? s : 1));
    double t[8];
    for (int64_t k = k0; k < k1; ++k) {
        for (int64_t r = 0; r < s; ++r) {
            const double e = net_residual(w + k * 24, mask + k * 8, x[k * s + r], y[k * s + r], t);
            terms[r] = e * e;
        }
        out[k] = hko_ordered_sum(terms, s);
    }
    free(terms);
}

HKO_EXPORT void hko_net_grad(const double* w, const double* mask, const double* x, const double* y,
                             const double* bar_out, int64_t s, double* grad, int64_t k0, int64_t k1) {
    double t[8];
    for (int64_t k = k0; k < k1; ++k) {
        const double* wk = w + k * 24;
        const double* mk = mask + k * 8;
        double acc[24];
        for (int j = 0; j < 24; ++j) acc[j] = 0.0;
        for (int64_t r = 0; r < s; ++r) {
            const double xi = x[k * s + r];
            const double lead = 2.0 * net_residual(wk, mk, xi, y[k * s + r], t) * bar_out[k];
            for (int h = 0; h < 8; ++h) {
                const double g = lead * mk[h] * wk[3 * h + 2] * (1.0 - t[h] * t[h]);
                acc[3 * h] += g * xi;
                acc[3 * h + 1] += g;
                acc[3 * h + 2] += lead * mk[h] * t[h];
            }
        }
        for (int j = 0; j < 24; ++j) grad[k * 24 + j] = acc[j];
    }
}

/* ---- config 5c: the keyed ordered scatter ---------------------------------
 * Reference hawk/emit/team.py:322-460 and hawk/_lane_bind.py:111-114:
 * chunks = clamp(n / cells, 1, 256), span = ceil(n / chunks); chunk b walks
 * its lanes in order, parts[key*chunks + b] += v (from 0); key -1 skipped,
 * another key outside [0, cells) sets status[1+b]; then each cell adds its
 * parts in chunk order from 0 and adds that onto target[cell]. */
HKO_EXPORT int hko_scatter_chunks(int64_t n, int64_t cells) {
    const int64_t fit = n / (cells < 1 ? 1 : cells);
    return (int)(fit < 1 ? 1 : (fit > 256 ? 256 : fit));
}

static void scatter_chunk(const int32_t* key, const double* v, int64_t n, int64_t cells, int chunks,
                          int b, double* parts, int32_t* status) {
    const int64_t span = (n + chunks - 1) / chunks;
    const int64_t lo = (int64_t)b * span;
    const int64_t hi = lo + span < n ? lo + span : n;
    for (int64_t r = lo; r < hi; ++r) {
        const int32_t k = key[r];
        if (k == -1) continue;
        if (k >= 0 && k < cells) parts[(int64_t)k * chunks + b] += v[r];
        else status[1 + b] = 1;
    }
}

static void scatter_cells(const double* parts, int64_t c_lo, int64_t c_hi, int chunks, double* target) {
    for (int64_t c = c_lo; c < c_hi; ++c) {
        double s = 0.0;
        for (int b = 0; b < chunks; ++b) s += parts[c * chunks + b];
        target[c] += s;
    }
}

/* parts: chunks*cells doubles of scratch; status: 257 int32. */
HKO_EXPORT void hko_ordered_scatter(const int32_t* key, const double* v, int64_t n, double* target,
                                    int64_t cells, double* parts, int32_t* status) {
    if (cells <= 0) return;
    const int chunks = hko_scatter_chunks(n, cells);
    memset(parts, 0, sizeof(double) * (size_t)chunks * (size_t)cells);
    status[0] = (int32_t)cells;
    for (int b = 0; b < 256; ++b) status[1 + b] = 0;
    for (int b = 0; b < chunks; ++b) scatter_chunk(key, v, n, cells, chunks, b, parts, status);
    scatter_cells(parts, 0, cells, chunks, target);
}

/* The keyed ordered scatter in the float32 mode (the walk's parts, the cells'
 * sums and the target are float; reference hawk/emit/team.py:322-460 over
 * `Real`).  parts: chunks*cells floats of scratch; status: 257 int32. */
HKO_EXPORT void hko_ordered_scatter_f32(const int32_t* key, const float* v, int64_t n, float* target,
                                        int64_t cells, float* parts, int32_t* status) {
    if (cells <= 0) return;
    const int chunks = hko_scatter_chunks(n, cells);
    memset(parts, 0, sizeof(float) * (size_t)chunks * (size_t)cells);
    status[0] = (int32_t)cells;
    for (int b = 0; b < 256; ++b) status[1 + b] = 0;
    const int64_t span = (n + chunks - 1) / chunks;
    for (int b = 0; b < chunks; ++b) {
        const int64_t lo = (int64_t)b * span;
        const int64_t hi = lo + span < n ? lo + span : n;
        for (int64_t r = lo; r < hi; ++r) {
            const int32_t k = key[r];
            if (k == -1) continue;
            if (k >= 0 && k < cells) parts[(int64_t)k * chunks + b] += v[r];
            else status[1 + b] = 1;
        }
    }
    for (int64_t c = 0; c < cells; ++c) {
        float acc = 0.0f;
        for (int b = 0; b < chunks; ++b) acc += parts[c * chunks + b];
        target[c] += acc;
    }
}

/* ---- config 3: two-body leapfrog, 32 kick-drift-kick substeps ------------
 * The kernel (tests/kernels.py `twobody`):
 *   r2 = dot(r, r); a = (-mu / (r2 * sqrt(r2))) * r
 *   vh = v + (0.5*dt) * a; r = r + dt * vh
 *   r2 = dot(r, r); a = (-mu / (r2 * sqrt(r2))) * r; v = vh + (0.5*dt) * a */
#define HKO_STEPS 32
#define HKO_DT 1e-3

static inline void accel(const double r[3], double mu, double a[3]) {
    const double r2 = ((r[0] * r[0]) + (r[1] * r[1])) + (r[2] * r[2]);
    const double s = -mu / (r2 * sqrt(r2));
    for (int c = 0; c < 3; ++c) a[c] = s * r[c];
}

static inline void substep(double r[3], double v[3], double mu) {
    double a[3], vh[3];
    accel(r, mu, a);
    for (int c = 0; c < 3; ++c) vh[c] = v[c] + ((0.5 * HKO_DT) * a[c]);
    for (int c = 0; c < 3; ++c) r[c] = r[c] + (HKO_DT * vh[c]);
    accel(r, mu, a);
    for (int c = 0; c < 3; ++c) v[c] = vh[c] + ((0.5 * HKO_DT) * a[c]);
}

HKO_EXPORT void hko_twobody(const double* r0, const double* v0, double mu, int64_t n, double* r_out,
                            double* v_out, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        double r[3], v[3];
        for (int c = 0; c < 3; ++c) { r[c] = r0[c * n + i]; v[c] = v0[c * n + i]; }
        for (int k = 0; k < HKO_STEPS; ++k) substep(r, v, mu);
        for (int c = 0; c < 3; ++c) { r_out[c * n + i] = r[c]; v_out[c * n + i] = v[c]; }
    }
}

/* The adjoint of a = s * r with s = -mu / (r2 * sqrt(r2)), r2 = dot(r, r):
 * given g = bar_a, accumulate into bar_r (held + new, in the reverse order of
 * the forward operations: the product's term, then the dot's two).
 * Rules of reference hawk/diff/rules.py:
 * mul(s, r): s gets sum(g*r), r gets g*s; div(-mu, q): q gets -(gs*s)/q;
 * mul(r2, sq): r2 gets gq*sq, sq gets gq*r2; sqrt: r2 gets gsq*(0.5/sq);
 * dot(r, r): r gets gr2*r twice. */
static inline void accel_vjp(const double r[3], double mu, const double g[3], double bar_r[3]) {
    const double r2 = ((r[0] * r[0]) + (r[1] * r[1])) + (r[2] * r[2]);
    const double sq = sqrt(r2);
    const double q = r2 * sq;
    const double s = -mu / q;
    const double gs = ((g[0] * r[0]) + (g[1] * r[1])) + (g[2] * r[2]);
    const double gq = -((gs * s) / q);
    const double gr2 = (gq * sq) + ((gq * r2) * (0.5 / sq));
    for (int c = 0; c < 3; ++c) bar_r[c] = ((bar_r[c] + (g[c] * s)) + (gr2 * r[c])) + (gr2 * r[c]);
}

/* Reverse of one substep from its start state (r, v) (replayed from the
 * tape): incoming (br, bv) are the adjoints of the substep's outputs and are
 * replaced by the adjoints of its inputs. */
static inline void substep_vjp(const double r_in[3], const double v_in[3], double mu, double br[3],
                               double bv[3]) {
    double a[3], vh[3], r1[3];
    accel(r_in, mu, a);
    for (int c = 0; c < 3; ++c) vh[c] = v_in[c] + ((0.5 * HKO_DT) * a[c]);
    for (int c = 0; c < 3; ++c) r1[c] = r_in[c] + (HKO_DT * vh[c]);
    /* v_out = vh + (0.5 dt) a(r1) */
    double bvh[3], ba1[3], br1[3];
    for (int c = 0; c < 3; ++c) { bvh[c] = bv[c]; ba1[c] = bv[c] * (0.5 * HKO_DT); br1[c] = br[c]; }
    accel_vjp(r1, mu, ba1, br1);
    /* r1 = r + dt * vh */
    double brn[3];
    for (int c = 0; c < 3; ++c) { brn[c] = br1[c]; bvh[c] += br1[c] * HKO_DT; }
    /* vh = v + (0.5 dt) a(r) */
    double ba0[3];
    for (int c = 0; c < 3; ++c) { bv[c] = bvh[c]; ba0[c] = bvh[c] * (0.5 * HKO_DT); }
    accel_vjp(r_in, mu, ba0, brn);
    for (int c = 0; c < 3; ++c) br[c] = brn[c];
}

HKO_EXPORT void hko_twobody_vjp(const double* r0, const double* v0, double mu, const double* bar_r,
                                const double* bar_v, int64_t n, double* bar_r0, double* bar_v0,
                                int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        double tr[HKO_STEPS][3], tv[HKO_STEPS][3], r[3], v[3], br[3], bv[3];
        for (int c = 0; c < 3; ++c) { r[c] = r0[c * n + i]; v[c] = v0[c * n + i]; }
        for (int k = 0; k < HKO_STEPS; ++k) {
            for (int c = 0; c < 3; ++c) { tr[k][c] = r[c]; tv[k][c] = v[c]; }
            substep(r, v, mu);
        }
        for (int c = 0; c < 3; ++c) { br[c] = bar_r[c * n + i]; bv[c] = bar_v[c * n + i]; }
        for (int k = HKO_STEPS - 1; k >= 0; --k) substep_vjp(tr[k], tv[k], mu, br, bv);
        for (int c = 0; c < 3; ++c) { bar_r0[c * n + i] = br[c]; bar_v0[c * n + i] = bv[c]; }
    }
}

/* ---- config 3 interchanged: the loop over samples inside the substep loop --
 * The reference host target's loop interchange for a rolled `for` body
 * (hawk/emit/host.py:961-1000, :1061 loop_interchange): a tile of samples
 * steps together, so each operation of a substep runs across the tile's
 * samples as one SIMD loop.  Per sample the operations and their order are
 * those of hko_twobody / hko_twobody_vjp, so the bits are theirs (sqrt and
 * division are correctly rounded in SIMD too); a ragged tail takes the
 * sample-by-sample loop. */
#define HKO_TILE 8

static inline void accel_tile(double r[3][HKO_TILE], double mu, double a[3][HKO_TILE]) {
    for (int t = 0; t < HKO_TILE; ++t) {
        const double r2 = ((r[0][t] * r[0][t]) + (r[1][t] * r[1][t])) + (r[2][t] * r[2][t]);
        const double s = -mu / (r2 * sqrt(r2));
        for (int c = 0; c < 3; ++c) a[c][t] = s * r[c][t];
    }
}

static inline void substep_tile(double r[3][HKO_TILE], double v[3][HKO_TILE], double mu) {
    double a[3][HKO_TILE], vh[3][HKO_TILE];
    accel_tile(r, mu, a);
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) vh[c][t] = v[c][t] + ((0.5 * HKO_DT) * a[c][t]);
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) r[c][t] = r[c][t] + (HKO_DT * vh[c][t]);
    accel_tile(r, mu, a);
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) v[c][t] = vh[c][t] + ((0.5 * HKO_DT) * a[c][t]);
}

HKO_EXPORT void hko_twobody_x(const double* r0, const double* v0, double mu, int64_t n, double* r_out,
                              double* v_out, int64_t base, int64_t count) {
    int64_t i = base;
    for (; i + HKO_TILE <= base + count; i += HKO_TILE) {
        double r[3][HKO_TILE], v[3][HKO_TILE];
        for (int c = 0; c < 3; ++c)
            for (int t = 0; t < HKO_TILE; ++t) { r[c][t] = r0[c * n + i + t]; v[c][t] = v0[c * n + i + t]; }
        for (int k = 0; k < HKO_STEPS; ++k) substep_tile(r, v, mu);
        for (int c = 0; c < 3; ++c)
            for (int t = 0; t < HKO_TILE; ++t) { r_out[c * n + i + t] = r[c][t]; v_out[c * n + i + t] = v[c][t]; }
    }
    hko_twobody(r0, v0, mu, n, r_out, v_out, i, base + count - i);
}

static inline void accel_vjp_tile(double r[3][HKO_TILE], double mu, double g[3][HKO_TILE],
                                  double bar_r[3][HKO_TILE]) {
    for (int t = 0; t < HKO_TILE; ++t) {
        const double r2 = ((r[0][t] * r[0][t]) + (r[1][t] * r[1][t])) + (r[2][t] * r[2][t]);
        const double sq = sqrt(r2);
        const double q = r2 * sq;
        const double s = -mu / q;
        const double gs = ((g[0][t] * r[0][t]) + (g[1][t] * r[1][t])) + (g[2][t] * r[2][t]);
        const double gq = -((gs * s) / q);
        const double gr2 = (gq * sq) + ((gq * r2) * (0.5 / sq));
        for (int c = 0; c < 3; ++c)
            bar_r[c][t] = ((bar_r[c][t] + (g[c][t] * s)) + (gr2 * r[c][t])) + (gr2 * r[c][t]);
    }
}

static inline void substep_vjp_tile(double r_in[3][HKO_TILE], double v_in[3][HKO_TILE], double mu,
                                    double br[3][HKO_TILE], double bv[3][HKO_TILE]) {
    double a[3][HKO_TILE], vh[3][HKO_TILE], r1[3][HKO_TILE];
    accel_tile(r_in, mu, a);
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) vh[c][t] = v_in[c][t] + ((0.5 * HKO_DT) * a[c][t]);
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) r1[c][t] = r_in[c][t] + (HKO_DT * vh[c][t]);
    double bvh[3][HKO_TILE], ba1[3][HKO_TILE], br1[3][HKO_TILE];
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) {
            bvh[c][t] = bv[c][t];
            ba1[c][t] = bv[c][t] * (0.5 * HKO_DT);
            br1[c][t] = br[c][t];
        }
    accel_vjp_tile(r1, mu, ba1, br1);
    double brn[3][HKO_TILE], ba0[3][HKO_TILE];
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) {
            brn[c][t] = br1[c][t];
            bvh[c][t] += br1[c][t] * HKO_DT;
        }
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) {
            bv[c][t] = bvh[c][t];
            ba0[c][t] = bvh[c][t] * (0.5 * HKO_DT);
        }
    accel_vjp_tile(r_in, mu, ba0, brn);
    for (int c = 0; c < 3; ++c)
        for (int t = 0; t < HKO_TILE; ++t) br[c][t] = brn[c][t];
}

HKO_EXPORT void hko_twobody_vjp_x(const double* r0, const double* v0, double mu, const double* bar_r,
                                  const double* bar_v, int64_t n, double* bar_r0, double* bar_v0,
                                  int64_t base, int64_t count) {
    int64_t i = base;
    for (; i + HKO_TILE <= base + count; i += HKO_TILE) {
        double tr[HKO_STEPS][3][HKO_TILE], tv[HKO_STEPS][3][HKO_TILE];
        double r[3][HKO_TILE], v[3][HKO_TILE], br[3][HKO_TILE], bv[3][HKO_TILE];
        for (int c = 0; c < 3; ++c)
            for (int t = 0; t < HKO_TILE; ++t) { r[c][t] = r0[c * n + i + t]; v[c][t] = v0[c * n + i + t]; }
        for (int k = 0; k < HKO_STEPS; ++k) {
            for (int c = 0; c < 3; ++c)
                for (int t = 0; t < HKO_TILE; ++t) { tr[k][c][t] = r[c][t]; tv[k][c][t] = v[c][t]; }
            substep_tile(r, v, mu);
        }
        for (int c = 0; c < 3; ++c)
            for (int t = 0; t < HKO_TILE; ++t) { br[c][t] = bar_r[c * n + i + t]; bv[c][t] = bar_v[c * n + i + t]; }
        for (int k = HKO_STEPS - 1; k >= 0; --k) substep_vjp_tile(tr[k], tv[k], mu, br, bv);
        for (int c = 0; c < 3; ++c)
            for (int t = 0; t < HKO_TILE; ++t) { bar_r0[c * n + i + t] = br[c][t]; bar_v0[c * n + i + t] = bv[c][t]; }
    }
    hko_twobody_vjp(r0, v0, mu, bar_r, bar_v, n, bar_r0, bar_v0, i, base + count - i);
}

/* ---- config 4a: 6x6 SPD Cholesky solve and its VJP -------------------------
 * Factor and solve in the operation order of reference
 * hawk/embedded/linalg.py:233-271 (`_chol`: the symmetrised entry
 * (0.5*a_ij) + (0.5*a_ji), row-ordered dot updates) and :443-536 (`_dot_rows`:
 * forward rows ascending, backward rows descending, each acc = src - sum in
 * column order, then / diagonal).  info != 0 gives zeros.
 * VJP (reference hawk/diff/linalg_rules.py:230-233): lam = cho_solve(L, bar_x);
 * bar_b = lam; bar_A = -((outer(lam, x) + outer(lam, x)^T) * 0.5). */
#define HKO_N 6

static int chol6(const double a[HKO_N][HKO_N], double l[HKO_N][HKO_N]) {
    int info = 0;
    for (int i = 0; i < HKO_N; ++i)
        for (int c = 0; c < HKO_N; ++c) l[i][c] = 0.0;
    for (int j = 0; j < HKO_N; ++j) {
        if (info != 0) continue;
        double d = (0.5 * a[j][j]) + (0.5 * a[j][j]);
        for (int k = 0; k < j; ++k) d = d - (l[j][k] * l[j][k]);
        if (d > 0.0) {
            const double ljj = sqrt(d);
            l[j][j] = ljj;
            for (int i = j + 1; i < HKO_N; ++i) {
                double acc = (0.5 * a[i][j]) + (0.5 * a[j][i]);
                for (int k = 0; k < j; ++k) acc = acc - (l[i][k] * l[j][k]);
                l[i][j] = acc / ljj;
            }
        } else {
            info = j + 1;
        }
    }
    return info;
}

static void cho_solve6(const double l[HKO_N][HKO_N], int info, const double b[HKO_N], double x[HKO_N]) {
    if (info != 0) {
        for (int i = 0; i < HKO_N; ++i) x[i] = 0.0;
        return;
    }
    for (int i = 0; i < HKO_N; ++i) {
        double acc = b[i];
        for (int j = 0; j < i; ++j) acc = acc - (l[i][j] * x[j]);
        x[i] = acc / l[i][i];
    }
    for (int r = 0; r < HKO_N; ++r) {
        const int i = HKO_N - 1 - r;
        double acc = x[i];
        for (int j = i + 1; j < HKO_N; ++j) acc = acc - (l[j][i] * x[j]);
        x[i] = acc / l[i][i];
    }
}

static void load6(const double* A, const double* b, int64_t n, int64_t i, double a[HKO_N][HKO_N],
                  double bb[HKO_N]) {
    for (int r = 0; r < HKO_N; ++r) {
        for (int c = 0; c < HKO_N; ++c) a[r][c] = A[(r * HKO_N + c) * n + i];
        bb[r] = b[r * n + i];
    }
}

HKO_EXPORT void hko_spd_solve(const double* A, const double* b, int64_t n, double* x_out, int64_t base,
                              int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        double a[HKO_N][HKO_N], l[HKO_N][HKO_N], bb[HKO_N], x[HKO_N];
        load6(A, b, n, i, a, bb);
        const int info = chol6(a, l);
        cho_solve6(l, info, bb, x);
        for (int r = 0; r < HKO_N; ++r) x_out[r * n + i] = x[r];
    }
}

HKO_EXPORT void hko_spd_solve_vjp(const double* A, const double* b, const double* bar_x, int64_t n,
                                  double* bar_A, double* bar_b, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        double a[HKO_N][HKO_N], l[HKO_N][HKO_N], bb[HKO_N], x[HKO_N], g[HKO_N], lam[HKO_N];
        load6(A, b, n, i, a, bb);
        const int info = chol6(a, l);
        cho_solve6(l, info, bb, x);
        for (int r = 0; r < HKO_N; ++r) g[r] = bar_x[r * n + i];
        cho_solve6(l, info, g, lam);
        for (int r = 0; r < HKO_N; ++r) {
            bar_b[r * n + i] = lam[r];
            for (int c = 0; c < HKO_N; ++c)
                bar_A[(r * HKO_N + c) * n + i] = -(((lam[r] * x[c]) + (lam[c] * x[r])) * 0.5);
        }
    }
}

/* ---- config 4b: fp32 16x16 product and its VJP --------------------------------
 * C_ij = sum_k A_ik B_kj added in k order (the rolled product); the VJP is
 * bar_A = bar_C B^T, bar_B = A^T bar_C (reference hawk/diff/rules.py `mm`),
 * each entry's products added in index order. */
#define HKO_M 16

HKO_EXPORT void hko_mm16(const float* A, const float* B, int64_t n, float* C, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        float a[HKO_M][HKO_M], b[HKO_M][HKO_M];
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                a[r][c] = A[(r * HKO_M + c) * n + i];
                b[r][c] = B[(r * HKO_M + c) * n + i];
            }
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                float acc = a[r][0] * b[0][c];
                for (int k = 1; k < HKO_M; ++k) acc = acc + (a[r][k] * b[k][c]);
                C[(r * HKO_M + c) * n + i] = acc;
            }
    }
}

HKO_EXPORT void hko_mm16_vjp(const float* A, const float* B, const float* bar_C, int64_t n, float* bar_A,
                             float* bar_B, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        float a[HKO_M][HKO_M], b[HKO_M][HKO_M], g[HKO_M][HKO_M];
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                a[r][c] = A[(r * HKO_M + c) * n + i];
                b[r][c] = B[(r * HKO_M + c) * n + i];
                g[r][c] = bar_C[(r * HKO_M + c) * n + i];
            }
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                float acc = g[r][0] * b[c][0];                 /* (g B^T)_rc = sum_k g_rk B_ck */
                for (int k = 1; k < HKO_M; ++k) acc = acc + (g[r][k] * b[c][k]);
                bar_A[(r * HKO_M + c) * n + i] = acc;
                float acc2 = a[0][r] * g[0][c];                /* (A^T g)_rc = sum_k A_kr g_kc */
                for (int k = 1; k < HKO_M; ++k) acc2 = acc2 + (a[k][r] * g[k][c]);
                bar_B[(r * HKO_M + c) * n + i] = acc2;
            }
    }
}

/* The same products in float64 (the reference's float64 mode builds the same
 * per-sample `mm`, reference hawk/targets/__init__.py:48-49): each element a
 * sequential sum over k of rounded products, from k = 0. */
HKO_EXPORT void hko_mm16_f64(const double* A, const double* B, int64_t n, double* C, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        double a[HKO_M][HKO_M], b[HKO_M][HKO_M];
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                a[r][c] = A[(r * HKO_M + c) * n + i];
                b[r][c] = B[(r * HKO_M + c) * n + i];
            }
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                double acc = a[r][0] * b[0][c];
                for (int k = 1; k < HKO_M; ++k) acc = acc + (a[r][k] * b[k][c]);
                C[(r * HKO_M + c) * n + i] = acc;
            }
    }
}

HKO_EXPORT void hko_mm16_vjp_f64(const double* A, const double* B, const double* bar_C, int64_t n, double* bar_A,
                                 double* bar_B, int64_t base, int64_t count) {
    for (int64_t i = base; i < base + count; ++i) {
        double a[HKO_M][HKO_M], b[HKO_M][HKO_M], g[HKO_M][HKO_M];
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                a[r][c] = A[(r * HKO_M + c) * n + i];
                b[r][c] = B[(r * HKO_M + c) * n + i];
                g[r][c] = bar_C[(r * HKO_M + c) * n + i];
            }
        for (int r = 0; r < HKO_M; ++r)
            for (int c = 0; c < HKO_M; ++c) {
                double acc = g[r][0] * b[c][0];
                for (int k = 1; k < HKO_M; ++k) acc = acc + (g[r][k] * b[c][k]);
                bar_A[(r * HKO_M + c) * n + i] = acc;
                double acc2 = a[0][r] * g[0][c];
                for (int k = 1; k < HKO_M; ++k) acc2 = acc2 + (a[k][r] * g[k][c]);
                bar_B[(r * HKO_M + c) * n + i] = acc2;
            }
    }
}

/* ---- the CPU baseline's tiling (eagle HostTeam shape) ------------------------
 * [0, n) is cut into T contiguous tiles, one thread per tile calling the
 * serial entry with its own (base, count) (reference hawk/emit/host.py:4-12);
 * the ordered sum runs one group per thread-slot and the ordered scatter one
 * chunk per thread-slot, each reproducing the serial bits. */
/* One launch of the oscillator that finishes its own sample (reference
 * tests/test_finish_own_sample.py:52-64 `osc_finish`, stepped by
 * hawk/trace/steps.py:1-20 when K > 1), over samples [base, base+count): a
 * sample whose mask is set is skipped; any other takes up to K steps of
 *     v' = v + dt*(-x);  x' = x + dt*v;  t' = t + dt
 * leaving after the step at which t' >= t_final (its values are that step's),
 * and then its mask is set.  Returns how many samples this launch finished
 * (the finished_count the reference adds to; :228-241 is its NumPy twin
 * with K = 1); `trips` (nullable) gets each sample's steps this launch (the
 * fast entries' reports, hawk/emit/cuda.py:692-702).  K <= 0 takes none. */
HKO_EXPORT int64_t hko_osc_launch(int64_t base, int64_t count, int K, double dt, const double* t_final, double* x,
                                  double* v, double* t, unsigned char* mask, int32_t* trips) {
    int64_t finished = 0;
    for (int64_t i = base; i < base + count; ++i) {
        if (mask[i]) { if (trips) trips[i] = 0; continue; }
        double xi = x[i], vi = v[i], ti = t[i];
        int done = 0, k = 0;
        for (; k < K && !done; ++k) {
            const double xn = xi + dt * vi;
            const double vn = vi + dt * (-xi);
            const double tn = ti + dt;
            xi = xn; vi = vn; ti = tn;
            done = tn >= t_final[i];
        }
        x[i] = xi; v[i] = vi; t[i] = ti;
        if (trips) trips[i] = k;          /* the steps this launch took of sample i */
        if (done) { mask[i] = 1; ++finished; }
    }
    return finished;
}

typedef struct {
    int which;
    const void* in0; const void* in1; const void* in2; const void* in3; const void* in4;
    void* out0; void* out1;
    double s0, s1;
    int64_t n, base, count;
    double* gp;
    int g_lo, g_hi;
    int64_t cells;
    int chunks;
    double* parts;
    int32_t* status;
} hko_job;

static void* job_main(void* arg) {
    hko_job* j = (hko_job*)arg;
    switch (j->which) {
        case 1: hko_scale((const double*)j->in0, j->s0, j->s1, (double*)j->out0, j->base, j->count); break;
        case 2: hko_energy((const double*)j->in0, j->n, (double*)j->out0, j->base, j->count); break;
        case 3: hko_energy_vjp((const double*)j->in0, (const double*)j->in1, j->n, (double*)j->out0,
                               j->base, j->count); break;
        case 4: hko_energy_jvp((const double*)j->in0, (const double*)j->in1, j->n, (double*)j->out0,
                               j->base, j->count); break;
        case 5: hko_chain((const double*)j->in0, (double*)j->out0, j->base, j->count); break;
        case 6:
            for (int g = j->g_lo; g < j->g_hi; ++g) j->gp[g] = group_part((const double*)j->in0, j->n, g);
            break;
        case 7:
            for (int b = j->g_lo; b < j->g_hi; ++b)
                scatter_chunk((const int32_t*)j->in0, (const double*)j->in1, j->n, j->cells, j->chunks, b,
                              j->parts, j->status);
            break;
        case 8: scatter_cells(j->parts, j->base, j->base + j->count, j->chunks, (double*)j->out0); break;
        case 9: hko_twobody_x((const double*)j->in0, (const double*)j->in1, j->s0, j->n, (double*)j->out0,
                              (double*)j->out1, j->base, j->count); break;
        case 10: hko_twobody_vjp_x((const double*)j->in0, (const double*)j->in1, j->s0, (const double*)j->in2,
                                   (const double*)j->in3, j->n, (double*)j->out0, (double*)j->out1, j->base,
                                   j->count); break;
        case 11: hko_spd_solve((const double*)j->in0, (const double*)j->in1, j->n, (double*)j->out0, j->base,
                               j->count); break;
        case 12: hko_spd_solve_vjp((const double*)j->in0, (const double*)j->in1, (const double*)j->in2, j->n,
                                   (double*)j->out0, (double*)j->out1, j->base, j->count); break;
        case 13: hko_mm16((const float*)j->in0, (const float*)j->in1, j->n, (float*)j->out0, j->base,
                          j->count); break;
        case 14: hko_mm16_vjp((const float*)j->in0, (const float*)j->in1, (const float*)j->in2, j->n,
                              (float*)j->out0, (float*)j->out1, j->base, j->count); break;
        case 15:   /* keys [base, base+count) of a keyed ordered sum, group = cells */
            for (int64_t k = j->base; k < j->base + j->count; ++k)
                ((double*)j->out0)[k] = hko_ordered_sum((const double*)j->in0 + k * j->cells, j->cells);
            break;
        case 16:   /* nets [base, base+count): their losses, s = cells samples each */
            hko_net_loss((const double*)j->in0, (const double*)j->in1, (const double*)j->in2,
                         (const double*)j->in3, j->cells, (double*)j->out0, j->base, j->base + j->count);
            break;
        case 21: hko_mm16_f64((const double*)j->in0, (const double*)j->in1, j->n, (double*)j->out0, j->base,
                              j->count); break;
        case 22: hko_mm16_vjp_f64((const double*)j->in0, (const double*)j->in1, (const double*)j->in2, j->n,
                                  (double*)j->out0, (double*)j->out1, j->base, j->count); break;
        case 18: hko_chain_members((const double*)j->in0, (double*)j->out0, (double*)j->out1, j->n, j->base,
                                   j->count); break;
        case 17:   /* nets [base, base+count): their gradients wrt w */
            hko_net_grad((const double*)j->in0, (const double*)j->in1, (const double*)j->in2,
                         (const double*)j->in3, (const double*)j->in4, j->cells, (double*)j->out0, j->base,
                         j->base + j->count);
            break;
        default: break;
    }
    return NULL;
}

static void run_jobs(hko_job* jobs, int t) {
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)t);
    for (int k = 0; k < t; ++k) pthread_create(&th[k], NULL, job_main, &jobs[k]);
    for (int k = 0; k < t; ++k) pthread_join(th[k], NULL);
    free(th);
}

/* One tiled run of a per-sample entry over [0, n) on `threads` threads. */
HKO_EXPORT void hko_tiled(int which, const void* in0, const void* in1, const void* in2, const void* in3,
                          void* out0, void* out1, double s0, double s1, int64_t n, int threads) {
    if (threads < 1) threads = 1;
    hko_job* jobs = (hko_job*)calloc((size_t)threads, sizeof(hko_job));
    const int64_t tile = (n + threads - 1) / threads;
    for (int k = 0; k < threads; ++k) {
        jobs[k].which = which;
        jobs[k].in0 = in0; jobs[k].in1 = in1; jobs[k].in2 = in2; jobs[k].in3 = in3;
        jobs[k].out0 = out0; jobs[k].out1 = out1; jobs[k].s0 = s0; jobs[k].s1 = s1; jobs[k].n = n;
        jobs[k].base = (int64_t)k * tile < n ? (int64_t)k * tile : n;
        const int64_t hi = jobs[k].base + tile < n ? jobs[k].base + tile : n;
        jobs[k].count = hi - jobs[k].base;
    }
    run_jobs(jobs, threads);
    free(jobs);
}

/* The ordered sum with its 64 groups spread over `threads` threads (same bits). */
HKO_EXPORT double hko_ordered_sum_threads(const double* u, int64_t n, int threads) {
    double gp[HKO_G];
    if (threads < 1) threads = 1;
    if (threads > HKO_G) threads = HKO_G;
    hko_job jobs[HKO_G];
    memset(jobs, 0, sizeof(jobs));
    const int per = (HKO_G + threads - 1) / threads;
    for (int k = 0; k < threads; ++k) {
        jobs[k].which = 6; jobs[k].in0 = u; jobs[k].n = n; jobs[k].gp = gp;
        jobs[k].g_lo = k * per < HKO_G ? k * per : HKO_G;
        jobs[k].g_hi = (k + 1) * per < HKO_G ? (k + 1) * per : HKO_G;
    }
    run_jobs(jobs, threads);
    return fold_groups(gp);
}

/* The keyed ordered sum with its keys spread over `threads` threads (same bits). */
HKO_EXPORT void hko_keyed_ordered_sum_threads(const double* u, int64_t n, int64_t group, double* out, int threads) {
    const int64_t keys = group > 0 ? n / group : 0;
    if (threads < 1) threads = 1;
    if (threads > keys) threads = keys > 0 ? (int)keys : 1;
    hko_job* jobs = (hko_job*)calloc((size_t)threads, sizeof(hko_job));
    const int64_t per = (keys + threads - 1) / threads;
    for (int k = 0; k < threads; ++k) {
        jobs[k].which = 15; jobs[k].in0 = u; jobs[k].out0 = out; jobs[k].cells = group;
        jobs[k].base = k * per < keys ? k * per : keys;
        jobs[k].count = ((k + 1) * per < keys ? (k + 1) * per : keys) - jobs[k].base;
    }
    run_jobs(jobs, threads);
    free(jobs);
}

/* The chain members over [0, n) in `threads` contiguous tiles (same bits). */
HKO_EXPORT void hko_chain_members_threads(const double* x, double* acc, double* y, int64_t n, int threads) {
    if (threads < 1) threads = 1;
    hko_job* jobs = (hko_job*)calloc((size_t)threads, sizeof(hko_job));
    const int64_t tile = (n + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        jobs[t].which = 18; jobs[t].in0 = x; jobs[t].out0 = acc; jobs[t].out1 = y; jobs[t].n = n;
        jobs[t].base = t * tile < n ? t * tile : n;
        jobs[t].count = ((t + 1) * tile < n ? (t + 1) * tile : n) - jobs[t].base;
    }
    run_jobs(jobs, threads);
    free(jobs);
}

/* The net axis's loss (which = 16) or gradient (17) with the nets spread over
 * `threads` threads (same bits). */
HKO_EXPORT void hko_net_threads(int which, const double* w, const double* mask, const double* x, const double* y,
                                const double* bar_out, int64_t k, int64_t s, double* out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > k) threads = k > 0 ? (int)k : 1;
    hko_job* jobs = (hko_job*)calloc((size_t)threads, sizeof(hko_job));
    const int64_t per = (k + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
        jobs[t].which = which; jobs[t].in0 = w; jobs[t].in1 = mask; jobs[t].in2 = x; jobs[t].in3 = y;
        jobs[t].in4 = bar_out; jobs[t].out0 = out; jobs[t].cells = s;
        jobs[t].base = t * per < k ? t * per : k;
        jobs[t].count = ((t + 1) * per < k ? (t + 1) * per : k) - jobs[t].base;
    }
    run_jobs(jobs, threads);
    free(jobs);
}

/* The ordered scatter with its chunks spread over `threads` threads (same bits). */
HKO_EXPORT void hko_ordered_scatter_threads(const int32_t* key, const double* v, int64_t n, double* target,
                                            int64_t cells, double* parts, int32_t* status, int threads) {
    if (cells <= 0) return;
    if (threads < 1) threads = 1;
    const int chunks = hko_scatter_chunks(n, cells);
    memset(parts, 0, sizeof(double) * (size_t)chunks * (size_t)cells);
    status[0] = (int32_t)cells;
    for (int b = 0; b < 256; ++b) status[1 + b] = 0;
    hko_job* jobs = (hko_job*)calloc((size_t)threads, sizeof(hko_job));
    const int per = (chunks + threads - 1) / threads;
    for (int k = 0; k < threads; ++k) {
        jobs[k].which = 7; jobs[k].in0 = key; jobs[k].in1 = v; jobs[k].n = n; jobs[k].cells = cells;
        jobs[k].chunks = chunks; jobs[k].parts = parts; jobs[k].status = status;
        jobs[k].g_lo = k * per < chunks ? k * per : chunks;
        jobs[k].g_hi = (k + 1) * per < chunks ? (k + 1) * per : chunks;
    }
    run_jobs(jobs, threads);
    const int64_t tile = (cells + threads - 1) / threads;
    for (int k = 0; k < threads; ++k) {
        jobs[k].which = 8; jobs[k].out0 = target;
        jobs[k].base = (int64_t)k * tile < cells ? (int64_t)k * tile : cells;
        const int64_t hi = jobs[k].base + tile < cells ? jobs[k].base + tile : cells;
        jobs[k].count = hi - jobs[k].base;
    }
    run_jobs(jobs, threads);
    free(jobs);
}
