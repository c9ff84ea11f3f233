/*
 * CPU oracle for the optimizer step after the MoE layer -- TEST
 * INFRASTRUCTURE ONLY.  Only tests/ load this library, and only to check
 * results; the product never links it.
 *
 * It restates one step of the name-keyed Adam of resihp/runtime/optim.py:32-46
 * (bit for bit the update of torch.optim.Adam(foreach=False), which the
 * reference asserts in tests/unit/test_state_basics.py:108-120), element by
 * element, in plain C built with -ffp-contract=off, with every fused
 * multiply-add written out.  The tensor operations of optim.py:41-46 evaluate,
 * per element and in this order (each pinned against torch's CPU kernels in
 * tests/test_oracle_adam.py):
 *
 *   g  = grad                                 (0 when the parameter has no grad)
 *   g  = fma(wd, p, g)                        g.add(p, alpha=wd), only if wd != 0
 *   m  = |w| < 0.5 ? fma(w, g - m, m)         exp_avg.lerp_(g, w), w = 1 - beta1
 *              : fma(w - 1, g - m, g)
 *   v  = v * b2                               exp_avg_sq.mul_(beta2)
 *   v  = fma(c * g, g, v)                     .addcmul_(g, g, value=c), c = 1 - beta2
 *   d  = sqrt(v)                              exp_avg_sq.sqrt()
 *   d  = d / bc2s                             / sqrt(1 - beta2^step)
 *   d  = d + eps                              .add_(eps)
 *   p  = p + (a * m) / d                      p.addcdiv_(m, d, value=a), a = -lr / (1 - beta1^step)
 *
 * The scalars are computed in double as Python computes them (bc1, bc2s, w,
 * c, a) and converted to the tensor's compute type: float for float32 and
 * bfloat16 tensors, double for float64 -- except the weight decay of a
 * bfloat16 tensor, which torch's add(alpha=) rounds to bfloat16 first.  A
 * bfloat16 tensor computes each operation in float and rounds its result to
 * bfloat16 (round to nearest even, NaN to 0x7fc0) before the next operation
 * reads it, as each torch operation writes a bfloat16 tensor.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static void scalars(double lr, double b1, double b2, int64_t step, double* w, double* c, double* bc2s, double* a) {
    const double bc1 = 1.0 - pow(b1, (double)step);
    *bc2s = sqrt(1.0 - pow(b2, (double)step));
    *w = 1.0 - b1;
    *c = 1.0 - b2;
    *a = -lr / bc1;
}

void oracle_adam_f64(double* p, const double* grad, double* m, double* v, int64_t n, double lr, double b1,
                     double b2, double eps, double wd, int64_t step) {
    double w, c, bc2s, a;
    scalars(lr, b1, b2, step, &w, &c, &bc2s, &a);
    for (int64_t i = 0; i < n; ++i) {
        double g = grad ? grad[i] : 0.0;
        if (wd != 0.0) g = fma(wd, p[i], g);
        m[i] = fabs(w) < 0.5 ? fma(w, g - m[i], m[i]) : fma(w - 1.0, g - m[i], g);
        double vv = v[i] * b2;
        vv = fma(c * g, g, vv);
        v[i] = vv;
        double d = sqrt(vv);
        d = d / bc2s;
        d = d + eps;
        p[i] = p[i] + (a * m[i]) / d;
    }
}

void oracle_adam_f32(float* p, const float* grad, float* m, float* v, int64_t n, double lr, double b1, double b2,
                     double eps, double wd, int64_t step) {
    double w, c, bc2s, a;
    scalars(lr, b1, b2, step, &w, &c, &bc2s, &a);
    const float wf = (float)w, cf = (float)c, b2f = (float)b2, bc2f = (float)bc2s, epsf = (float)eps, af = (float)a,
                wdf = (float)wd;
    for (int64_t i = 0; i < n; ++i) {
        float g = grad ? grad[i] : 0.0f;
        if (wd != 0.0) g = fmaf(wdf, p[i], g);
        m[i] = fabsf(wf) < 0.5f ? fmaf(wf, g - m[i], m[i]) : fmaf(wf - 1.0f, g - m[i], g);
        float vv = v[i] * b2f;
        vv = fmaf(cf * g, g, vv);
        v[i] = vv;
        float d = sqrtf(vv);
        d = d / bc2f;
        d = d + epsf;
        p[i] = p[i] + (af * m[i]) / d;
    }
}

static float bf(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* float -> bfloat16, round to nearest even; NaN -> 0x7fc0 (torch's c10::BFloat16). */
static uint16_t rbf(float f) {
    if (f != f) return 0x7fc0;
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

void oracle_adam_bf16(uint16_t* p, const uint16_t* grad, uint16_t* m, uint16_t* v, int64_t n, double lr, double b1,
                      double b2, double eps, double wd, int64_t step) {
    double w, c, bc2s, a;
    scalars(lr, b1, b2, step, &w, &c, &bc2s, &a);
    const float wf = (float)w, cf = (float)c, b2f = (float)b2, bc2f = (float)bc2s, epsf = (float)eps, af = (float)a,
                wdf = bf(rbf((float)wd));
    for (int64_t i = 0; i < n; ++i) {
        uint16_t g = grad ? grad[i] : 0;
        const float pf = bf(p[i]);
        if (wd != 0.0) g = rbf(fmaf(wdf, pf, bf(g)));
        const float gf = bf(g), mf = bf(m[i]);
        m[i] = rbf(fabsf(wf) < 0.5f ? fmaf(wf, gf - mf, mf) : fmaf(wf - 1.0f, gf - mf, gf));
        const uint16_t v1 = rbf(bf(v[i]) * b2f);
        v[i] = rbf(fmaf(cf * gf, gf, bf(v1)));
        uint16_t d = rbf(sqrtf(bf(v[i])));
        d = rbf(bf(d) / bc2f);
        d = rbf(bf(d) + epsf);
        p[i] = rbf(pf + (af * bf(m[i])) / bf(d));
    }
}
