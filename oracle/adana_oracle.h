/*
 * adana_oracle.h -- declarations of the CPU restatement in adana_oracle.c.
 *
 * TEST INFRASTRUCTURE ONLY (see adana_oracle.c): used by tests/ and the
 * bench's CPU baseline, never by the product.
 */
#ifndef ADANA_ORACLE_H
#define ADANA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    float a;        /* alpha = fp32(delta / (delta + t)), double divide      */
    float oma;      /* fp32(1 - a)                                           */
    float s;        /* fp32(t)                                               */
    float eps;      /* fp32(epsilon)                                         */
    float pw;       /* ADana: fp32((1 + s) ** (1 - kappa)), binary64 pow     */
    float min_p;    /* Star: fp32(1 / (1 + s))                               */
    float clip;     /* fp32(clipsnr)                                         */
    int32_t has_clip;
    float c3;       /* fp32(-lr) * fp32(gamma_3_factor)                      */
    float cg2;      /* fp32(-lr)                                             */
    float opw;      /* fp32(1 + wd_factor)                                   */
    float star_exp; /* fp32(1 - kappa): exponent of the per-element pow      */
    int32_t pow_mode; /* ATen's pow(Tensor, Scalar) specialisation, below     */
    int32_t compiled; /* 1: torch.compile's (Inductor's) forms of lerp and the
                         second-moment update, bfloat16 rounding only where a
                         tensor is stored; 0: the ATen eager ops              */
    int32_t pow_int;  /* POW_INT: the integer exponent                         */
    int32_t foreach;  /* 1: the reference's use_foreach=True path (below)       */
    float g3f;      /* foreach: fp32(gamma_3_factor)                         */
    float lr;       /* foreach: fp32(lr), both g2 and g3                     */
    float wdf;      /* foreach: the weight-decay factor (p += p * wdf)       */
} adana_oracle_scalars;

/* Manau's Dana-Star-MK4 branch (src/optim/manau.py:556-613): its scalars
 * are the branch's Python floats rounded to binary32 where they meet float32
 * tensors (tensor-scalar operands, full_like). */
typedef struct {
    float a;        /* fp32(alpha)                                        */
    float oma;      /* fp32(1 - alpha), binary64 difference               */
    float s;        /* fp32(step)                                         */
    float eps;      /* fp32(epsilon)                                      */
    float min_p;    /* fp32(1 / (1 + step)), binary64 quotient            */
    float clip;     /* fp32(clipsnr)                                      */
    float lr;       /* fp32(lr)                                           */
    float wdf;      /* fp32(1 - wd/(1+step/wd_ts)*lr) or fp32(1 - wd*lr)  */
    float e[3];     /* fp32 exponents: 1-kappa, 2 mk4B + 1, 2 (-mk4A - mk4B) */
    int32_t mode[3];/* their ATen specialisations                         */
    int32_t has_wd; /* weight_decay != 0                                  */
    int32_t reserved;
} adana_oracle_manau_scalars;

/* One step over n elements of one tensor; diag receives the binary64 sums
 * of alpha_factor, g^2, mfac and m^2. */
void adana_oracle_adana_step(int64_t n, float *p, const float *g, float *m, float *v,
                             const adana_oracle_scalars *sc, double diag[4]);
void adana_oracle_star_step(int64_t n, float *p, const float *g, float *m, float *v,
                            float *tau, const adana_oracle_scalars *sc, double diag[4]);
void adana_oracle_manau_step(int64_t n, float *p, const float *g, float *m, float *v, float *tau,
                             const adana_oracle_manau_scalars *sc, double diag[4]);
void adana_oracle_master_step(int64_t n, int32_t star, float *master, uint16_t *p16,
                              const uint16_t *g16, float *m, float *v, float *tau,
                              const adana_oracle_scalars *sc, double diag[4]);
void adana_oracle_step_g16(int64_t n, int32_t star, float *p, const uint16_t *g16, float *m,
                           float *v, float *tau, const adana_oracle_scalars *sc, double diag[4]);
void adana_oracle_step_bf16(int64_t n, int32_t star, uint16_t *p, const uint16_t *g, uint16_t *m,
                            uint16_t *v, uint16_t *tau, const adana_oracle_scalars *sc, double diag[4]);
void adana_oracle_f32_to_bf16(int64_t n, const float *x, uint16_t *y);
int adana_oracle_abi_version(void);
void adana_oracle_set_threads(int n);
int adana_oracle_get_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* ADANA_ORACLE_H */
