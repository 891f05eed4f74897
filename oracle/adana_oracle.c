/*
 * adana_oracle.c -- CPU restatement of the ADana-family optimizer step.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (adana_amd/) links, loads
 * or calls this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg do, and only as the checker / the timed CPU baseline.
 *
 * What it restates (reference = mlexpos/adana):
 *   adana_oracle_adana_step  <- ADana._update_param_compiled
 *                               src/optim/adana.py:100-151
 *   adana_oracle_star_step   <- DANA_STAR_MK4._update_param_compiled
 *                               src/optim/dana_star_mk4.py:136-203
 *   adana_oracle_manau_step  <- Manau.step's Dana-Star-MK4 branch
 *                               src/optim/manau.py:556-613
 *   adana_oracle_step_bf16   <- both updates on bfloat16 parameters (the
 *                               reference's own bfloat16 path, every op
 *                               rounded to bfloat16; rules below)
 *   adana_oracle_scalars.foreach: the same entry points step the
 *                               reference's use_foreach=True path instead
 *                               (src/optim/adana.py:229-370,
 *                               src/optim/dana_star_mk4.py:298-536)
 *
 * Arithmetic contract (the oracle of record):
 *   - every tensor op of the reference is one IEEE-754 binary32 operation,
 *     correctly rounded, in the reference's op order; no contraction
 *     (built with -ffp-contract=off);
 *   - the two composite ops the reference uses have two forms, chosen by
 *     adana_oracle_scalars.compiled:
 *       eager (the update run as ATen ops, torch.compile disabled): single-
 *       rounded FMAs, as torch 2.10's CPU kernels compute them (probed bitwise)
 *         lerp(a, b, w)          = |w| < 0.5 ? fma(w, b-a, a) : fma(w-1, b-a, b)
 *         addcmul(s, t, t, val)  = fma(val*t, t, s)
 *       compiled (the reference's default path, torch.compile, adana.py:72-79,
 *       dana_star_mk4.py:88-96): Inductor's decompositions, every product and
 *       sum rounded on its own (its C++ is built with -ffp-contract=off)
 *         lerp(a, b, w)          = (|w| < 0.5 ? w : w-1) * (b-a) + (|w| < 0.5 ? a : b)
 *         v*(1-val) + addcmul    = v*(1-val) + (t*t)*val
 *     (read from Inductor's generated code for a restatement of the update
 *     as the same torch ops, and pinned by the reference's compiled runs);
 *   - Dana-Star's per-element pow(et, 1-kappa) takes the exponent rounded to
 *     binary32 (the vectorised ATen path does) and is evaluated in binary64,
 *     then rounded once to binary32;
 *   - sign(x) is 0 for x == +-0 and NaN; clamp / relu propagate NaN.
 *
 * Per-tensor diagnostics (reference :146-151 / :198-203) are accumulated in
 * binary64: sum(alpha_factor), sum(g^2), sum(mfac), sum(m^2).
 *
 * Parity pins for this file (see tests/test_oracle.py):
 *   - golden vectors written by the reference's own step() in this container
 *     (tests/golden/make_golden.py): m, v bit-exact; tau and p within a few
 *     ulp (the reference's CPU sqrt/pow are Sleef approximations);
 *   - closed forms for a constant gradient (m_t = g(1-Pi_t), v_t = g^2(1-Pi_t));
 *   - invariants (state independent of p, clipsnr=inf == no clip, kappa=1 =>
 *     pow == 1, weight_decay=0 => opw == 1) and a binary64 brute-force loop.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "adana_oracle.h"


/* pow(Tensor, Scalar) specialisations, chosen on the binary64 exponent.
 * ATen (eager): 0 -> ones, 1 -> copy, 0.5 -> sqrt, -0.5 -> 1/sqrt, -1 -> 1/x,
 * 2 -> x*x, 3 -> x*x*x, -2 -> 1/(x*x); anything else a general pow.
 * Inductor (compiled): 0 -> ones, 1 -> copy, 0.5 -> sqrt, another integer k
 * with |k| < 32 -> POW_INT (products, below); anything else a general pow. */
enum { POW_GENERAL = 0, POW_ONE, POW_SQRT, POW_RSQRT, POW_RECIP, POW_SQUARE, POW_CUBE, POW_INVSQ, POW_IDENTITY,
       POW_INT };

/* x ** k as Inductor's pow_recursive expands it (torch/_inductor/
 * lowering.py): for k < 0 the powers of 1/x; x**(2j) = x**j * x**j and
 * x**(2j+1) = (x**j * x**j) * x, each product rounded to binary32. */
static float o_pow_int(float x, int32_t k) {
    if (k < 0) {
        x = 1.0f / x;
        k = -k;
    }
    if (k == 0) return 1.0f;
    if (k == 1) return x;
    float r = o_pow_int(x, k / 2);
    r = r * r;
    return (k % 2) ? r * x : r;
}

/* x ** e by ATen's specialisation `mode` (chosen on the binary64 exponent);
 * any other exponent: binary64 pow of the binary32 exponent, rounded once. */
static inline float o_pow_mode(float x, float e, int32_t mode) {
    switch (mode) {
    case POW_ONE: return 1.0f;
    case POW_IDENTITY: return x;
    case POW_SQRT: return sqrtf(x);
    case POW_RSQRT: return 1.0f / sqrtf(x);
    case POW_RECIP: return 1.0f / x;
    case POW_SQUARE: return x * x;
    case POW_CUBE: return (x * x) * x;
    case POW_INVSQ: return 1.0f / (x * x);
    default: return (float)pow((double)x, (double)e);
    }
}

static inline float o_pow(float x, const adana_oracle_scalars *sc) {
    switch (sc->pow_mode) {
    case POW_INT: return o_pow_int(x, sc->pow_int);
    case POW_ONE: return 1.0f;
    case POW_IDENTITY: return x;
    case POW_SQRT: return sqrtf(x);
    case POW_RSQRT: return 1.0f / sqrtf(x);
    case POW_RECIP: return 1.0f / x;
    case POW_SQUARE: return x * x;
    case POW_CUBE: return (x * x) * x;
    case POW_INVSQ: return 1.0f / (x * x);
    default: return (float)pow((double)x, (double)sc->star_exp);
    }
}

static inline float o_lerp(float self, float end, float w, int32_t compiled) {
    float d = end - self;
    if (compiled) {
        const int small = fabsf(w) < 0.5f;
        return (small ? w : w - 1.0f) * d + (small ? self : end);
    }
    return (fabsf(w) < 0.5f) ? fmaf(w, d, self) : fmaf(w - 1.0f, d, end);
}
/* v.mul_(1 - alpha).addcmul_(g, g, value=alpha) (adana.py:104) */
static inline float o_ema2(float v, float g, const adana_oracle_scalars *sc) {
    if (sc->compiled) return v * sc->oma + (g * g) * sc->a;
    return fmaf(sc->a * g, g, v * sc->oma);
}
static inline float o_sign(float x) { return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f); }
static inline float o_clamp_max(float x, float c) { return x > c ? c : x; }
static inline float o_clamp_min(float x, float c) { return x < c ? c : x; }
static inline float o_relu(float x) { return x < 0.0f ? 0.0f : x; }

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}
/* Round-to-nearest-even binary32 -> bfloat16 (NaN kept quiet). */
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float o_maximum(float a, float b) {   /* torch.maximum: NaN propagates */
    if (a != a) return a;
    if (b != b) return b;
    return a < b ? b : a;
}

/* One ADana / Dana-MK4 element (src/optim/adana.py:101-143). */
static inline float adana_elem(float p, float g, float *mp, float *vp,
                               const adana_oracle_scalars *sc, double acc[4]) {
    float m = o_lerp(*mp, g, sc->a, sc->compiled);           /* :101 */
    float v = o_ema2(*vp, g, sc);                            /* :104 mul_, addcmul_ */
    float se = sqrtf(v) + sc->eps;                           /* :107 */
    float nt = 1.0f / se;                                    /* :110 */
    float mn = fabsf(m) * nt;                                /* :111, :115 */
    float af = sc->pw * mn;                                  /* :119/:123 */
    if (sc->has_clip) af = o_clamp_max(af, sc->clip);        /* :118-121 */
    float inner = o_sign(m) * af + m * nt;                   /* :126 */
    float g3t = sc->c3 * inner;
    float g2t = (sc->cg2 * g) * nt;                          /* :129 */
    float u = g2t + g3t;                                     /* :132 */
    p = p + u;                                               /* :135 */
    p = p * sc->opw;                                         /* :143 */
    *mp = m;
    *vp = v;
    acc[0] += (double)af;
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mn;
    acc[3] += (double)m * (double)m;
    return p;
}

/* One Dana-Star / Dana-Star-MK4 element (src/optim/dana_star_mk4.py:137-195). */
static inline float star_elem(float p, float g, float *mp, float *vp, float *tp,
                              const adana_oracle_scalars *sc, double acc[4]) {
    float m = o_lerp(*mp, g, sc->a, sc->compiled);           /* :137 */
    float v = o_ema2(*vp, g, sc);                            /* :140 */
    float se = sqrtf(v) + sc->eps;                           /* :143 */
    float ag = fabsf(g);                                     /* :147 */
    float tu = ag / (ag + se);                               /* :148 */
    float tau = o_lerp(*tp, tu, sc->a, sc->compiled);        /* :149 */
    float ct = o_clamp_max(tau, 0.5f);                       /* :152 */
    float pe = ct / (1.0f - ct);                             /* :153 */
    float tr = sc->min_p + o_relu(pe - sc->min_p);           /* :154-156 */
    float et = o_clamp_min(tau * sc->s, 1.0f);               /* :159 */
    float nt = sqrtf(tr) / se;                               /* :163-164 */
    float mnt = fabsf(m) * nt;                               /* :165 */
    float mf = mnt / tr;                                     /* :167 */
    float pw = o_pow(et, sc);                                /* :170 / :174 */
    float af = pw * mf;
    if (sc->has_clip) af = o_clamp_max(af, sc->clip);        /* :169-172 */
    float inner = o_sign(m) * (tr * af + mnt);               /* :177 */
    float g3t = sc->c3 * inner;
    float g2t = (sc->cg2 * g) * nt;                          /* :180 */
    float u = g2t + g3t;                                     /* :183 */
    p = p + u;                                               /* :186 */
    p = p * sc->opw;                                         /* :195 */
    *mp = m;
    *vp = v;
    *tp = tau;
    acc[0] += (double)af;
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mf;
    acc[3] += (double)m * (double)m;
    return p;
}


/* One element of Manau's Dana-Star-MK4 branch (src/optim/manau.py:566-613).
 * ATen's add_(x, alpha=a) and addcmul_(g, g, value=a) are single-rounded
 * FMAs (probed bitwise against torch 2.10's CPU kernels). */
static inline float manau_elem(float p, float g, float *mp, float *vp, float *tp,
                               const adana_oracle_manau_scalars *sc, double acc[4]) {
    float m = fmaf(g, sc->a, *mp * sc->oma);                 /* :567 */
    float v = fmaf(sc->a * g, g, *vp * sc->oma);             /* :569 */
    float ag = fabsf(g);
    float sv = sqrtf(v);
    float tu = ag / ((ag + sv) + sc->eps);                   /* :572, _tau_updater :292-299 */
    float tau = fmaf(tu, sc->a, *tp * sc->oma);              /* :573 */
    float ct = o_clamp_max(tau, 0.5f);                       /* _tau_reg :277-282 */
    float pe = ct / (1.0f - ct);
    float tr = o_maximum(pe, sc->min_p);
    float et = o_maximum(tau * sc->s, 1.0f);                 /* _effective_time :288-290 */
    float nt = sqrtf(tr) / (sv + sc->eps);                   /* _norm_term :301-310 */
    float mfac = (nt * fabsf(m)) / tr;                       /* :583 */
    float af = (o_pow_mode(et, sc->e[0], sc->mode[0]) *      /* :584-589 */
                o_pow_mode(mfac, sc->e[1], sc->mode[1])) * o_pow_mode(nt, sc->e[2], sc->mode[2]);
    af = o_clamp_max(af, sc->clip);
    float i1 = (tr * o_sign(m)) * af;                        /* :590-593 */
    float i2 = (1.0f * m) * nt;
    float g3 = sc->lr * (i1 + i2);
    float g2 = (sc->lr * g) * nt;                            /* :600 */
    float u = -(g2 + g3);                                    /* :603 */
    if (sc->has_wd) p = p * sc->wdf;                         /* :606-610 */
    p = p + u;                                               /* :613 */
    *mp = m;
    *vp = v;
    *tp = tau;
    acc[0] += (double)af;                                    /* :595-598 */
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mfac;
    acc[3] += (double)m * (double)m;
    return p;
}

/* ---------------------------------------------------------------------------
 * The reference's own bfloat16 path: bfloat16 parameters make m, v and tau
 * bfloat16 too (zeros_like(p), src/optim/adana.py:191-195;
 * src/optim/dana_star_mk4.py:251-255), and every tensor op of the update
 * rounds its result to bfloat16 after computing in binary32, as ATen's CPU
 * kernels do.  How each op meets its binary32 0-d and Python-scalar
 * operands was probed op by op against torch 2.10's CPU kernels and is
 * pinned by the reference's own bfloat16 run (tests/golden/, the bf16_eager fixtures):
 *   - lerp_(end, w), w a float32 0-d tensor: w is rounded to bfloat16 first;
 *   - mul / div with the 0-d tensor as the second operand (v.mul_(1 - a),
 *     tau * step, p.mul_(1 + wd)): binary32 value as it is;
 *   - the 0-d tensor as the first operand ((-g2) * grad, (-g3)*gf * ...,
 *     pow * mfac in ADana, min_p + relu(...)), or any add / sub with a
 *     scalar (add_(epsilon), pe - min_p): the scalar rounded to bfloat16;
 *   - addcmul_(g, g, value=a): (a * g) * g + v in binary32, a unrounded;
 *   - Dana-Star's pow(et, 1 - kappa): the exponent rounded to bfloat16;
 *   - clamp(x, max=c): c rounded to bfloat16.
 * ------------------------------------------------------------------------- */
static inline float rb(float x) { return bf16_to_f32(f32_to_bf16(x)); }

/* x ** e16 (e16 already bfloat16) by ATen's specialisation, rounded once to
 * binary32 and then to bfloat16. */
static inline float o_pow16(float x, float e16, int32_t mode) { return rb(o_pow_mode(x, e16, mode)); }

static inline float adana_elem16(float p, float g, float *mp, float *vp, const adana_oracle_scalars *sc,
                                 double acc[4]) {
    const float a16 = rb(sc->a);
    float m = rb(o_lerp(*mp, g, a16, 0));                    /* :101 */
    float v = rb(*vp * sc->oma);                             /* :104 mul_ */
    v = rb(fmaf(sc->a * g, g, v));                           /* :104 addcmul_ */
    float se = rb(rb(sqrtf(v)) + rb(sc->eps));               /* :107 */
    float nt = rb(1.0f / se);                                /* :110 */
    float mn = rb(fabsf(m) * nt);                            /* :111, :115 */
    float af = rb(rb(sc->pw) * mn);                          /* :119/:123 */
    if (sc->has_clip) af = o_clamp_max(af, rb(sc->clip));
    float inner = rb(o_sign(m) * af + rb(m * nt));           /* :126 */
    float g3t = rb(rb(sc->c3) * inner);
    float g2t = rb(rb(rb(sc->cg2) * g) * nt);                /* :129 */
    p = rb(p + rb(g2t + g3t));                               /* :132-135 */
    p = rb(p * sc->opw);                                     /* :143 */
    *mp = m;
    *vp = v;
    acc[0] += (double)af;
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mn;
    acc[3] += (double)m * (double)m;
    return p;
}

static inline float star_elem16(float p, float g, float *mp, float *vp, float *tp,
                                const adana_oracle_scalars *sc, double acc[4]) {
    const float a16 = rb(sc->a), minp16 = rb(sc->min_p);
    float m = rb(o_lerp(*mp, g, a16, 0));                    /* :137 */
    float v = rb(*vp * sc->oma);                             /* :140 */
    v = rb(fmaf(sc->a * g, g, v));
    float se = rb(rb(sqrtf(v)) + rb(sc->eps));               /* :143 */
    float ag = fabsf(g);                                     /* :147 */
    float tu = rb(ag / rb(ag + se));                         /* :148 */
    float tau = rb(o_lerp(*tp, tu, a16, 0));                 /* :149 */
    float ct = o_clamp_max(tau, 0.5f);                       /* :152 */
    float pe = rb(ct / rb(1.0f - ct));                       /* :153 */
    float tr = rb(minp16 + o_relu(rb(pe - minp16)));         /* :154-156 */
    float et = o_clamp_min(rb(tau * sc->s), 1.0f);           /* :159 */
    float nt = rb(rb(sqrtf(tr)) / se);                       /* :163-164 */
    float mnt = rb(fabsf(m) * nt);                           /* :165 */
    float mf = rb(mnt / tr);                                 /* :167 */
    float af = rb(o_pow16(et, rb(sc->star_exp), sc->pow_mode) * mf);   /* :170 / :174 */
    if (sc->has_clip) af = o_clamp_max(af, rb(sc->clip));
    float inner = o_sign(m) * rb(rb(tr * af) + mnt);         /* :177 */
    float g3t = rb(rb(sc->c3) * inner);
    float g2t = rb(rb(rb(sc->cg2) * g) * nt);                /* :180 */
    p = rb(p + rb(g2t + g3t));                               /* :183-186 */
    p = rb(p * sc->opw);                                     /* :195 */
    *mp = m;
    *vp = v;
    *tp = tau;
    acc[0] += (double)af;
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mf;
    acc[3] += (double)m * (double)m;
    return p;
}

/* ---------------------------------------------------------------------------
 * The reference's foreach path (use_foreach=True): _foreach_compute_kernel_impl,
 * src/optim/adana.py:310-370 and src/optim/dana_star_mk4.py:395-536, one
 * element of one tensor, one binary32 operation per torch._foreach_* op in
 * that order.  Its forms differ from the per-tensor update's: no addcmul
 * (v * (1 - a) + (g * g) * a), tau_reg = maximum(p_estimate, min_p),
 * mfac = nt * (|m| / tau_reg), g3 scaled as (inner * gamma_3_factor) * lr,
 * g2 = (g * nt) * lr, p - (g2 + g3) and then p + p * wdf.  Its lerps are
 * ATen's in both of the reference's modes (torch.compile keeps a foreach
 * lerp with a list of weight tensors as the ATen kernel), so under
 * torch.compile on bfloat16 tensors (l16) m and tau come out of that kernel
 * rounded to bfloat16, tau's lerp reads the tau update rounded to bfloat16,
 * and everything else is binary32 from those values; the alpha factor and
 * mfac that the diagnostics average are the bfloat16 tensors the kernel
 * returns.  Scalars: alpha = fp32(delta) / (fp32(delta) + step) and
 * min_p = 1 / (step + 1) in binary32, step in the parameters' dtype
 * (adana.py:258-259, dana_star_mk4.py:455-456); wdf from adana.py:357-365.
 * ------------------------------------------------------------------------- */
static inline float fe_lerp(float self, float end, const adana_oracle_scalars *sc, int l16) {
    return l16 ? rb(o_lerp(self, end, rb(sc->a), 0)) : o_lerp(self, end, sc->a, 0);
}

static inline float adana_elem_fe(float p, float g, float *mp, float *vp, const adana_oracle_scalars *sc,
                                  int l16, double acc[4]) {
    float m = fe_lerp(*mp, g, sc, l16);                      /* _foreach_lerp_ */
    float v = *vp * sc->oma + (g * g) * sc->a;               /* mul_, mul, mul, add_ */
    float nt = 1.0f / (sqrtf(v) + sc->eps);                  /* sqrt, add, reciprocal */
    float mf = fabsf(m) * nt;                                /* abs, mul */
    float af = sc->pw * mf;                                  /* pow (0-d), mul */
    if (sc->has_clip) af = o_clamp_max(af, sc->clip);
    float inner = o_sign(m) * af + m * nt;                   /* sign, mul, mul, add */
    float g3t = (inner * sc->g3f) * sc->lr;                  /* mul_(gamma_3_factor), mul(g3) */
    float g2t = (g * nt) * sc->lr;                           /* mul, mul(g2) */
    p = p - (g2t + g3t);                                     /* add, neg_, add_ */
    p = p + p * sc->wdf;                                     /* mul, add_ */
    *mp = m;
    *vp = v;
    acc[0] += (double)(l16 ? rb(af) : af);
    acc[1] += (double)g * (double)g;
    acc[2] += (double)(l16 ? rb(mf) : mf);
    acc[3] += (double)m * (double)m;
    return p;
}

static inline float star_elem_fe(float p, float g, float *mp, float *vp, float *tp,
                                 const adana_oracle_scalars *sc, int l16, double acc[4]) {
    float m = fe_lerp(*mp, g, sc, l16);                      /* _foreach_lerp_ */
    float v = *vp * sc->oma + (g * g) * sc->a;               /* mul_, mul, mul, add_ */
    float sv = sqrtf(v);                                     /* sqrt_vs */
    float ag = fabsf(g);
    float tu = ag / ((ag + sv) + sc->eps);                   /* add, add_(epsilon), div */
    float tau = fe_lerp(*tp, l16 ? rb(tu) : tu, sc, l16);    /* _foreach_lerp_ */
    float ct = o_clamp_max(tau, 0.5f);                       /* clamp */
    float pe = ct / (1.0f - ct);                             /* neg, add_(1.0), div */
    float tr = o_maximum(pe, sc->min_p);                     /* maximum */
    float et = o_maximum(tau * sc->s, 1.0f);                 /* mul, maximum(., ones) */
    float nt = sqrtf(tr) / (sv + sc->eps);                   /* sqrt, add, div */
    float mf = nt * (fabsf(m) / tr);                         /* abs, div, mul */
    float af = o_pow(et, sc) * mf;                           /* pow, mul */
    if (sc->has_clip) af = o_clamp_max(af, sc->clip);
    float inner = (tr * o_sign(m)) * af + m * nt;            /* sign, mul, mul, mul, add */
    float g3t = (inner * sc->g3f) * sc->lr;                  /* mul_(gamma_3_factor), mul(g3) */
    float g2t = (g * nt) * sc->lr;                           /* mul, mul(g2) */
    p = p - (g2t + g3t);                                     /* add, neg_, add_ */
    p = p + p * sc->wdf;                                     /* mul, add_ */
    *mp = m;
    *vp = v;
    *tp = tau;
    acc[0] += (double)(l16 ? rb(af) : af);
    acc[1] += (double)g * (double)g;
    acc[2] += (double)(l16 ? rb(mf) : mf);
    acc[3] += (double)m * (double)m;
    return p;
}

/* The foreach path's eager ops on bfloat16 tensors (torch.compile off):
 * every op rounded to bfloat16 as ATen's kernels do, with the operand rules
 * of the per-tensor eager path above, and two of the foreach ops' own: an
 * in-place _foreach_mul_ by a Python scalar takes the scalar rounded to
 * bfloat16 (gamma_3_factor), an out-of-place one does not; a Python scalar
 * added (epsilon) is rounded to bfloat16 in every form.  A 0-d float32
 * tensor second in a multiplication (1 - alpha, alpha, lr, the weight-decay
 * factor) keeps its binary32 value.  Scalars (oracle.foreach_scalars with a
 * bfloat16 step, eager): min_p and ADana's power are the bfloat16 0-d
 * results, wdf the float32 0-d product (or, without decay, the bfloat16
 * copy).  (Probed op by op against torch 2.10, pinned by the reference's
 * own run, tests/golden/<case>.bf16_foreach_eager.npz.) */
static inline float adana_elem_fe16e(float p, float g, float *mp, float *vp, const adana_oracle_scalars *sc,
                                     double acc[4]) {
    const float a16 = rb(sc->a), e16 = rb(sc->eps);
    float m = rb(o_lerp(*mp, g, a16, 0));                    /* _foreach_lerp_ */
    float v = rb(*vp * sc->oma);                             /* _foreach_mul_(vs, 1 - alpha) */
    v = rb(v + rb(rb(g * g) * sc->a));                       /* mul, mul, add_ */
    float nt = rb(1.0f / rb(rb(sqrtf(v)) + e16));            /* sqrt, add(eps), reciprocal */
    float mf = rb(fabsf(m) * nt);
    float af = rb(sc->pw * mf);                              /* pow (0-d, bfloat16), mul */
    if (sc->has_clip) af = o_clamp_max(af, rb(sc->clip));
    float g3i = rb(rb(o_sign(m) * af) + rb(m * nt));         /* sign, mul, mul, add */
    g3i = rb(g3i * rb(sc->g3f));                             /* _foreach_mul_(., gamma_3_factor) */
    float upd = rb(rb(g3i * sc->lr) + rb(rb(g * nt) * sc->lr));   /* mul(g3), mul, mul(g2), add */
    p = rb(p - upd);                                         /* neg_, add_ */
    p = rb(p + rb(p * sc->wdf));                             /* mul, add_ */
    *mp = m;
    *vp = v;
    acc[0] += (double)af;
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mf;
    acc[3] += (double)m * (double)m;
    return p;
}

static inline float star_elem_fe16e(float p, float g, float *mp, float *vp, float *tp,
                                    const adana_oracle_scalars *sc, double acc[4]) {
    const float a16 = rb(sc->a), e16 = rb(sc->eps);
    float m = rb(o_lerp(*mp, g, a16, 0));                    /* _foreach_lerp_ */
    float v = rb(*vp * sc->oma);                             /* _foreach_mul_(vs, 1 - alpha) */
    v = rb(v + rb(rb(g * g) * sc->a));                       /* mul, mul, add_ */
    float sv = rb(sqrtf(v));
    float ag = fabsf(g);
    float tu = rb(ag / rb(rb(ag + sv) + e16));               /* add, add_(eps), div */
    float tau = rb(o_lerp(*tp, tu, a16, 0));                 /* _foreach_lerp_ */
    float ct = o_clamp_max(tau, 0.5f);
    float pe = rb(ct / rb(1.0f - ct));                       /* neg, add_(1.0), div */
    float tr = o_maximum(pe, sc->min_p);                     /* maximum */
    float et = o_maximum(rb(tau * sc->s), 1.0f);             /* mul, maximum(., ones) */
    float nt = rb(rb(sqrtf(tr)) / rb(sv + e16));             /* sqrt, add(eps), div */
    float mf = rb(nt * rb(fabsf(m) / tr));                   /* abs, div, mul */
    float af = rb(o_pow16(et, rb(sc->star_exp), sc->pow_mode) * mf);   /* pow, mul */
    if (sc->has_clip) af = o_clamp_max(af, rb(sc->clip));
    float g3i = rb(rb(rb(tr * o_sign(m)) * af) + rb(m * nt)); /* sign, mul, mul, mul, add */
    g3i = rb(g3i * rb(sc->g3f));                             /* _foreach_mul_(., gamma_3_factor) */
    float upd = rb(rb(g3i * sc->lr) + rb(rb(g * nt) * sc->lr));   /* mul(g3), mul, mul(g2), add */
    p = rb(p - upd);                                         /* neg_, add_ */
    p = rb(p + rb(p * sc->wdf));                             /* mul, add_ */
    *mp = m;
    *vp = v;
    *tp = tau;
    acc[0] += (double)af;
    acc[1] += (double)g * (double)g;
    acc[2] += (double)mf;
    acc[3] += (double)m * (double)m;
    return p;
}

/* Parallel element loops.  Element results do not depend on the thread
 * count; the binary64 diagnostic sums may differ in the last bits. */
#define DIAG_LOOP(BODY)                                                        \
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;                             \
    _Pragma("omp parallel for schedule(static) reduction(+:s0,s1,s2,s3) if(n > 65536)") \
    for (int64_t i = 0; i < n; ++i) {                                          \
        double acc[4] = {0.0, 0.0, 0.0, 0.0};                                  \
        BODY;                                                                  \
        s0 += acc[0]; s1 += acc[1]; s2 += acc[2]; s3 += acc[3];                \
    }                                                                          \
    diag[0] = s0; diag[1] = s1; diag[2] = s2; diag[3] = s3;

/* The element update of one float32 tensor (per-tensor or foreach forms). */
static inline float elem32(int32_t star, float p, float g, float *mp, float *vp, float *tp,
                           const adana_oracle_scalars *sc, double acc[4]) {
    if (sc->foreach)
        return star ? star_elem_fe(p, g, mp, vp, tp, sc, 0, acc) : adana_elem_fe(p, g, mp, vp, sc, 0, acc);
    return star ? star_elem(p, g, mp, vp, tp, sc, acc) : adana_elem(p, g, mp, vp, sc, acc);
}

void adana_oracle_adana_step(int64_t n, float *p, const float *g, float *m, float *v,
                             const adana_oracle_scalars *sc, double diag[4]) {
    DIAG_LOOP(p[i] = elem32(0, p[i], g[i], &m[i], &v[i], NULL, sc, acc))
}

void adana_oracle_star_step(int64_t n, float *p, const float *g, float *m, float *v,
                            float *tau, const adana_oracle_scalars *sc, double diag[4]) {
    DIAG_LOOP(p[i] = elem32(1, p[i], g[i], &m[i], &v[i], &tau[i], sc, acc))
}

void adana_oracle_manau_step(int64_t n, float *p, const float *g, float *m, float *v, float *tau,
                             const adana_oracle_manau_scalars *sc, double diag[4]) {
    DIAG_LOOP(p[i] = manau_elem(p[i], g[i], &m[i], &v[i], &tau[i], sc, acc))
}

/* bf16-parameter mode (an extension; the reference has no master weights):
 * the fp32 master copy is the parameter of the fp32 math, the gradient is
 * bf16 widened exactly, and the bf16 parameter is RNE(master). tau may be
 * NULL for the ADana variants. */
void adana_oracle_master_step(int64_t n, int32_t star, float *master, uint16_t *p16,
                              const uint16_t *g16, float *m, float *v, float *tau,
                              const adana_oracle_scalars *sc, double diag[4]) {
    DIAG_LOOP(master[i] = elem32(star, master[i], bf16_to_f32(g16[i]), &m[i], &v[i], star ? &tau[i] : NULL,
                                 sc, acc);
              p16[i] = f32_to_bf16(master[i]))
}

/* fp32 parameters with bf16 gradients (extension, same math). */
void adana_oracle_step_g16(int64_t n, int32_t star, float *p, const uint16_t *g16, float *m,
                           float *v, float *tau, const adana_oracle_scalars *sc,
                           double diag[4]) {
    DIAG_LOOP(p[i] = elem32(star, p[i], bf16_to_f32(g16[i]), &m[i], &v[i], star ? &tau[i] : NULL, sc, acc))
}

/* The reference's bfloat16 path: p, g, m, v and tau all bfloat16 (tau may
 * be NULL for the ADana variants).  Compiled (sc->compiled): Inductor loads
 * the bfloat16 tensors as binary32, runs the whole update in binary32 (the
 * compiled forms above, scalars unrounded) and rounds only the four stored
 * results to bfloat16 (round to nearest even).  Eager: every op rounded to
 * bfloat16 as ATen's bfloat16 kernels do (adana_elem16, star_elem16). */
void adana_oracle_step_bf16(int64_t n, int32_t star, uint16_t *p, const uint16_t *g, uint16_t *m,
                            uint16_t *v, uint16_t *tau, const adana_oracle_scalars *sc, double diag[4]) {
    if (sc->foreach && !sc->compiled && star) {     /* the foreach path's eager ops */
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]); float tt = bf16_to_f32(tau[i]);
                  p[i] = f32_to_bf16(star_elem_fe16e(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, &tt, sc, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv); tau[i] = f32_to_bf16(tt))
    } else if (sc->foreach && !sc->compiled) {
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]);
                  p[i] = f32_to_bf16(adana_elem_fe16e(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, sc, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv))
    } else if (sc->foreach && star) {      /* the foreach path under torch.compile */
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]); float tt = bf16_to_f32(tau[i]);
                  p[i] = f32_to_bf16(star_elem_fe(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, &tt, sc, 1, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv); tau[i] = f32_to_bf16(tt))
    } else if (sc->foreach) {
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]);
                  p[i] = f32_to_bf16(adana_elem_fe(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, sc, 1, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv))
    } else if (sc->compiled && star) {
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]); float tt = bf16_to_f32(tau[i]);
                  p[i] = f32_to_bf16(star_elem(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, &tt, sc, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv); tau[i] = f32_to_bf16(tt))
    } else if (sc->compiled) {
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]);
                  p[i] = f32_to_bf16(adana_elem(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, sc, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv))
    } else if (star) {
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]); float tt = bf16_to_f32(tau[i]);
                  p[i] = f32_to_bf16(star_elem16(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, &tt, sc, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv); tau[i] = f32_to_bf16(tt))
    } else {
        DIAG_LOOP(float mm = bf16_to_f32(m[i]); float vv = bf16_to_f32(v[i]);
                  p[i] = f32_to_bf16(adana_elem16(bf16_to_f32(p[i]), bf16_to_f32(g[i]), &mm, &vv, sc, acc));
                  m[i] = f32_to_bf16(mm); v[i] = f32_to_bf16(vv))
    }
}

void adana_oracle_f32_to_bf16(int64_t n, const float *x, uint16_t *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = f32_to_bf16(x[i]);
}

int adana_oracle_abi_version(void) { return 3; }

/* Thread count of the parallel loops (the CPU baseline reports it). */
#include <omp.h>
void adana_oracle_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }
int adana_oracle_get_threads(void) { return omp_get_max_threads(); }
