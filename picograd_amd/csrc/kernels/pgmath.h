/*
 * Scalar f32 math shared by the hand-written kernels and the JIT-generated
 * ones (the JIT embeds this file's text ahead of every program it compiles).
 *
 * Written for the VALU budget of an HBM-bound kernel on gfx950: with packed
 * FP32 off, one lane-instruction costs as much as ~2 bytes of HBM traffic at
 * peak, so libm-grade erff (~60 instructions) would make a fused GELU
 * backward compute-bound.  Accuracy target: the f32 grads of the path are
 * held to 1e-5 relative error (the reference itself builds with
 * -ffast-math); every function here stays within a few f32 ulps of the
 * exact value over its whole domain.
 *
 * PGM_EXP2 and PGM_RCP are the hardware 2^x and 1/x (v_exp_f32, v_rcp_f32,
 * both within 1 ulp); a host build of this header (the CPU unit test) maps
 * them to exp2f and a division.
 */
#ifndef PGK_PGMATH_H
#define PGK_PGMATH_H

#if defined(__HIP_DEVICE_COMPILE__) || defined(__HIPCC_RTC__)
#define PGM_FN __device__ __forceinline__
#define PGM_EXP2(x) __builtin_amdgcn_exp2f(x)
#define PGM_RCP(x) __builtin_amdgcn_rcpf(x)
#elif defined(__HIPCC__)
#define PGM_FN __host__ __device__ inline
#define PGM_EXP2(x) exp2f(x)
#define PGM_RCP(x) (1.0f / (x))
#else
#include <math.h>
#define PGM_FN static inline
#define PGM_EXP2(x) exp2f(x)
#define PGM_RCP(x) (1.0f / (x))
#endif

/* e^x as 2^(x log2 e).  The rounding of x*log2(e) costs |x| * 2^-24 * ln 2
 * relative, below 1e-6 for every x whose e^x is a normal f32. */
PGM_FN float pgm_exp(float x) { return PGM_EXP2(x * 1.44269504089f); }

/* logistic sigmoid 1 / (1 + e^-x) (the reference's activations.c:149-160) */
PGM_FN float pgm_sigmoid(float x) { return PGM_RCP(1.0f + pgm_exp(-x)); }

/*
 * Standard normal density phi(z) and distribution Phi(z), the two halves of
 * GELU (activations.c:166-173: gelu(z) = z * Phi(z) with Phi written as
 * 0.5 (1 + erf(z / sqrt 2))) and of its derivative (autograd.c:794-801:
 * Phi(z) + z phi(z)).
 *
 * Phi(-|z|) = phi(z) * t * P(t),  t = 1 / (1 + p |z|),
 * the form of Abramowitz & Stegun 26.2.17 with a degree-8 P fitted for this
 * file (iteratively reweighted least squares towards minimax on z in
 * [0, 14]): relative error 1.8e-8 in exact arithmetic, below f32 rounding.
 * The exponential phi needs anyway is the only transcendental; the tail
 * Phi(-|z|) comes out with relative (not just absolute) accuracy, and
 * Phi(z) for z > 0 is 1 - Phi(-z).
 */
PGM_FN float pgm_phi_tail(float z, float *density)
{
    const float p = 0.263464875f;
    float e = PGM_EXP2(z * z * -0.721347520444f); /* exp(-z^2 / 2) */
    float phi = e * 0.398942280401f;              /* 1 / sqrt(2 pi) */
    float t = PGM_RCP(1.0f + p * fabsf(z));
    float P = 0.0780001506f;
    P = P * t - 0.372467279f;
    P = P * t + 0.579365075f;
    P = P * t - 0.325497687f;
    P = P * t + 0.367844224f;
    P = P * t + 0.142426163f;
    P = P * t + 0.258060277f;
    P = P * t + 0.262051702f;
    P = P * t + 0.263531536f;
    *density = phi;
    return phi * t * P;
}

PGM_FN float pgm_Phi(float z, float *density)
{
    float q = pgm_phi_tail(z, density);
    return z < 0.0f ? q : 1.0f - q;
}

PGM_FN float pgm_gelu(float z)
{
    float d;
    return z * pgm_Phi(z, &d);
}

PGM_FN float pgm_gelu_grad(float z)
{
    float d;
    float P = pgm_Phi(z, &d);
    return P + z * d;
}

#endif
