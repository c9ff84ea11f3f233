/*
 * CPU oracle for the MoE routing path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only to check results.  The product never links it.
 *
 * It restates, in plain C with IEEE single/double arithmetic and no
 * floating-point contraction (built with -ffp-contract=off), the routing
 * contract the HIP kernels implement bit for bit:
 *
 *   router logits   resihp/runtime/moe.py:76  (logits = x @ router.t())
 *                   evaluated in a fixed order: the hidden dimension is cut
 *                   into segments of SEG = min(256, h) elements; each segment
 *                   is one fused-multiply-add chain starting at +0 in
 *                   ascending element order; the segment sums are added left
 *                   to right.
 *   selection       resihp/runtime/moe.py:77  (topk(logits + bias, k)),
 *                   descending key, ties to the lowest expert id, NaN keys
 *                   ranked as -inf.  Sigmoid scoring selects on
 *                   sigmoid(logit) + bias (DeepSeek-V3 style extension).
 *   gates           resihp/runtime/moe.py:79  (softmax over the *unbiased*
 *                   selected logits), sums taken in slot order; sigmoid gates
 *                   are the selected scores, optionally normalised by their
 *                   slot-order sum, times a scale.
 *   counts/offsets  resihp/runtime/moe.py:94,192  (bincount)
 *   permutation     resihp/runtime/moe.py:97,199-205 on one device: pairs
 *                   (token, slot) sorted stably by expert id, i.e. expert
 *                   major, then flat pair index t*k+j ascending.
 *
 * exp() is evaluated by one published method, shared with the kernels so that
 * both produce identical bits: Cody-Waite range reduction (n = rint(x*log2 e),
 * r = x - n*ln2_hi - n*ln2_lo, with the fdlibm split of ln 2) followed by the
 * Taylor polynomial of exp(r) in Horner form (degree 7 in single precision,
 * degree 13 in double precision) and an exact scaling by 2^n.  Arguments below
 * -87 (single) or -708 (double) return +0, so the scaling never produces a
 * subnormal; above ln(FLT_MAX) / ln(DBL_MAX) the result is +inf.
 *
 * Parity pins (tests/test_oracle_route.py): exp against libm to < 2 ulp;
 * logits against float64 dot products; selection against brute force over all
 * k-subsets and against a stable sort; planted ties; dispatch against numpy's
 * stable argsort and bincount.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ---------------------------------------------------------------- exp --- */

float oracle_expf(float x) {
    if (x != x) return x;
    if (x > 0x1.62e42ep+6f) return INFINITY;          /* > ln(FLT_MAX)  */
    if (x < -87.0f) return 0.0f;                      /* result stays normal above */
    float n = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-n, 0x1.62e4p-1f, x);
    r = fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0x1p-1f);
    p = fmaf(p, r, 0x1p+0f);
    p = fmaf(p, r, 0x1p+0f);
    return ldexpf(p, (int)n);
}

double oracle_exp(double x) {
    if (x != x) return x;
    if (x > 0x1.62e42fefa39efp+9) return INFINITY;    /* > ln(DBL_MAX)  */
    if (x < -708.0) return 0.0;                       /* result stays normal above */
    double n = rint(x * 0x1.71547652b82fep+0);
    double r = fma(-n, 0x1.62e42feep-1, x);
    r = fma(-n, 0x1.a39ef35793c76p-33, r);
    static const double c[14] = {
        0x1p+0, 0x1p+0, 0x1p-1, 0x1.5555555555555p-3, 0x1.5555555555555p-5,
        0x1.1111111111111p-7, 0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-13,
        0x1.a01a01a01a01ap-16, 0x1.71de3a556c734p-19, 0x1.27e4fb7789f5cp-22,
        0x1.ae64567f544e4p-26, 0x1.1eed8eff8d898p-29, 0x1.6124613a86d09p-33};
    double p = c[13];
    for (int i = 12; i >= 0; --i) p = fma(p, r, c[i]);
    return ldexp(p, (int)n);
}

static float sigmoidf_rhp(float x) { return 1.0f / (1.0f + oracle_expf(-x)); }
static double sigmoid_rhp(double x) { return 1.0 / (1.0 + oracle_exp(-x)); }

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* x_kind: 0 = float64, 1 = float32, 2 = bfloat16 (raw uint16 bits). */
static inline float load_xf(const void* x, int kind, int64_t i) {
    if (kind == 2) return bf16_to_f32(((const uint16_t*)x)[i]);
    return ((const float*)x)[i];
}

int oracle_router_segment(int h) { return h < 256 ? h : 256; }

/* Router logits in single precision: x is float32 or bfloat16, w is float32. */
int oracle_router_logits_f32(const void* x, int x_kind, const float* w, int64_t T, int h, int E,
                             float* logits) {
    int seg = oracle_router_segment(h);
    if (h <= 0 || h % 8 || h % seg) return -1;
    for (int64_t t = 0; t < T; ++t) {
        for (int e = 0; e < E; ++e) {
            float total = 0.0f;
            for (int s = 0; s < h / seg; ++s) {
                float acc = 0.0f;
                for (int i = s * seg; i < (s + 1) * seg; ++i)
                    acc = fmaf(load_xf(x, x_kind, t * h + i), w[(int64_t)e * h + i], acc);
                total = (s == 0) ? acc : total + acc;
            }
            logits[t * E + e] = total;
        }
    }
    return 0;
}

/* Router logits in double precision: x and w are float64. */
int oracle_router_logits_f64(const double* x, const double* w, int64_t T, int h, int E, double* logits) {
    int seg = oracle_router_segment(h);
    if (h <= 0 || h % 8 || h % seg) return -1;
    for (int64_t t = 0; t < T; ++t) {
        for (int e = 0; e < E; ++e) {
            double total = 0.0;
            for (int s = 0; s < h / seg; ++s) {
                double acc = 0.0;
                for (int i = s * seg; i < (s + 1) * seg; ++i)
                    acc = fma(x[t * h + i], w[(int64_t)e * h + i], acc);
                total = (s == 0) ? acc : total + acc;
            }
            logits[t * E + e] = total;
        }
    }
    return 0;
}

/* score: 0 = softmax over the selected logits, 1 = sigmoid. */
#define DEFINE_TOPK(T, SUF, SIGMOID, EXP)                                                         \
    int oracle_topk_##SUF(const T* logits, const T* bias, int64_t n_tok, int E, int k, int score, \
                          int normalize, T scale, int32_t* topi, T* gates) {                      \
        if (k <= 0 || k > E || E > 1024) return -1;                                               \
        T key[1024];                                                                              \
        unsigned char taken[1024];                                                                \
        for (int64_t t = 0; t < n_tok; ++t) {                                                     \
            const T* l = logits + t * E;                                                          \
            for (int e = 0; e < E; ++e) {                                                         \
                T v = score ? SIGMOID(l[e]) : l[e];                                               \
                if (bias) v = v + bias[e];                                                        \
                key[e] = (v != v) ? (T)(-INFINITY) : v;                                           \
                taken[e] = 0;                                                                     \
            }                                                                                     \
            for (int j = 0; j < k; ++j) {                                                         \
                int best = -1;                                                                    \
                for (int e = 0; e < E; ++e) {                                                     \
                    if (taken[e]) continue;                                                       \
                    if (best < 0 || key[e] > key[best]) best = e;                                 \
                }                                                                                 \
                taken[best] = 1;                                                                  \
                topi[t * k + j] = best;                                                           \
            }                                                                                     \
            T* g = gates + t * k;                                                                 \
            const int32_t* sel = topi + t * k;                                                    \
            if (score == 0) {                                                                     \
                T m = l[sel[0]];                                                                  \
                for (int j = 1; j < k; ++j) m = (l[sel[j]] > m) ? l[sel[j]] : m;                  \
                T s = 0;                                                                          \
                for (int j = 0; j < k; ++j) {                                                     \
                    g[j] = EXP(l[sel[j]] - m);                                                    \
                    s = (j == 0) ? g[j] : s + g[j];                                               \
                }                                                                                 \
                for (int j = 0; j < k; ++j) g[j] = (g[j] / s) * scale;                            \
            } else {                                                                              \
                T s = 0;                                                                          \
                for (int j = 0; j < k; ++j) {                                                     \
                    g[j] = SIGMOID(l[sel[j]]);                                                    \
                    s = (j == 0) ? g[j] : s + g[j];                                               \
                }                                                                                 \
                for (int j = 0; j < k; ++j) g[j] = (normalize ? g[j] / s : g[j]) * scale;         \
            }                                                                                     \
        }                                                                                         \
        return 0;                                                                                 \
    }

DEFINE_TOPK(float, f32, sigmoidf_rhp, oracle_expf)
DEFINE_TOPK(double, f64, sigmoid_rhp, oracle_exp)

/* Source rank of token t when [0, T) is cut by even_split(T, n_src)
 * (resihp/utils/intervals.py:17-30: the first T % n_src parts get one extra). */
static int source_of(int64_t t, int64_t T, int n_src) {
    int64_t base = T / n_src, rem = T % n_src;
    int64_t big = rem * (base + 1);
    if (t < big) return (int)(t / (base + 1));
    return (int)(rem + (t - big) / base);
}

/*
 * Dispatch plan for the local experts [e0, e1):
 *   counts[e]       pairs routed to expert e, for every e in [0, E); counts[E]
 *                   counts expert ids outside [0, E) (they are dropped)
 *   offsets[i]      exclusive prefix of counts[e0 + i], i in [0, e1 - e0]
 *   src_counts[s*L + i]  local pairs of expert e0 + i whose token lies in
 *                   source s of even_split(T, n_src), L = e1 - e0
 *   perm[r]         flat pair index t*k + j of local row r
 *   pair_row[p]     local row of pair p, or -1 when its expert is not local
 */
int oracle_dispatch(const int32_t* topi, int64_t T, int k, int E, int e0, int e1, int n_src,
                    int32_t* counts, int32_t* offsets, int32_t* src_counts, int32_t* perm,
                    int32_t* pair_row) {
    if (E <= 0 || k <= 0 || e0 < 0 || e1 > E || e0 > e1 || n_src <= 0) return -1;
    int L = e1 - e0;
    int64_t P = T * k;
    memset(counts, 0, sizeof(int32_t) * (size_t)(E + 1));
    memset(src_counts, 0, sizeof(int32_t) * (size_t)n_src * (size_t)L);
    for (int64_t p = 0; p < P; ++p) {
        int e = topi[p];
        if (e < 0 || e >= E) {
            counts[E]++;
            continue;
        }
        counts[e]++;
        if (e >= e0 && e < e1) src_counts[(int64_t)source_of(p / k, T, n_src) * L + (e - e0)]++;
    }
    offsets[0] = 0;
    for (int i = 0; i < L; ++i) offsets[i + 1] = offsets[i] + counts[e0 + i];
    int32_t fill[1024];
    if (L > 1024) return -1;
    for (int i = 0; i < L; ++i) fill[i] = offsets[i];
    for (int64_t p = 0; p < P; ++p) {
        int e = topi[p];
        if (e < e0 || e >= e1) {
            pair_row[p] = -1;
            continue;
        }
        int r = fill[e - e0]++;
        perm[r] = (int32_t)p;
        pair_row[p] = r;
    }
    return 0;
}
