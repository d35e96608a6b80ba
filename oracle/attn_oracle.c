/*
 * CPU oracle for the causal self-attention forward/backward of Filipeak/gpt.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP product path, never part
 * of it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load this library.
 *
 * The fp32 functions restate the reference CPU backend's algorithm step by
 * step, in the same loop nesting and the same summation order, so that with
 * the same compiler flags they reproduce its outputs bit for bit:
 *   forward  = src/backend/cpu/cpu_backend.cpp:289-356
 *   backward = src/backend/cpu/cpu_backend.cpp:358-437
 * The loop order has to match for that bit-exactness; the code is written
 * independently of the reference's text.
 *
 * Pinning (tests/test_oracle.py): bit-exact against the reference's own
 * CPUBackend built from /root/reference into oracle/_ref (when present);
 * closed forms (T=1, identical keys -> prefix means, LSE = c + ln(i+1));
 * invariants (shift of K, causality, sum_j dK_j = 0, sum_j dV_j = sum_i dO_i);
 * an independent dense fp64 numpy restatement; fp64 finite differences of
 * <O, dO>; and torch's scaled_dot_product_attention(is_causal=True) autograd.
 */
#include "attn_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Row-major offsets: element (b, t, col) of a [B, T, W] tensor. */
static inline long at3(long b, long t, long col, long T, long W)
{
    return (b * T + t) * W + col;
}

/* One generator for both precisions: REAL is the element type, EXPF/LOGF/SQRTF
 * the matching libm calls, LOWEST the most negative finite value. */
#define ORACLE_FORWARD(NAME, REAL, EXPF, LOGF, SQRTF, LOWEST)                          \
    void NAME(REAL *y, REAL *lse, const REAL *qkv, int B, int T, int C, int H)         \
    {                                                                                  \
        const long d = C / H;                                                          \
        const long W = 3L * C;                                                         \
        const REAL scale = (REAL)1 / SQRTF((REAL)d);                                   \
        REAL *row = (REAL *)malloc((size_t)(T > 0 ? T : 1) * sizeof(REAL));            \
        for (long b = 0; b < B; ++b)                                                   \
            for (long h = 0; h < H; ++h)                                               \
            {                                                                          \
                const REAL *q = qkv + at3(b, 0, h * d, T, W);                          \
                const REAL *k = qkv + at3(b, 0, C + h * d, T, W);                      \
                const REAL *v = qkv + at3(b, 0, 2L * C + h * d, T, W);                 \
                for (long i = 0; i < T; ++i)                                           \
                {                                                                      \
                    /* scaled scores of row i against keys 0..i; running max */        \
                    REAL m = LOWEST;                                                   \
                    for (long j = 0; j <= i; ++j)                                      \
                    {                                                                  \
                        REAL s = 0;                                                    \
                        for (long e = 0; e < d; ++e)                                   \
                            s += q[i * W + e] * k[j * W + e];                          \
                        s *= scale;                                                    \
                        row[j] = s;                                                    \
                        if (s > m)                                                     \
                            m = s;                                                     \
                    }                                                                  \
                    /* unnormalised probabilities and their sum, j ascending */        \
                    REAL l = 0;                                                        \
                    for (long j = 0; j <= i; ++j)                                      \
                    {                                                                  \
                        row[j] = EXPF(row[j] - m);                                     \
                        l += row[j];                                                   \
                    }                                                                  \
                    /* y = (sum_j p_j v_j) / l, one output column at a time */         \
                    for (long e = 0; e < d; ++e)                                       \
                    {                                                                  \
                        REAL acc = 0;                                                  \
                        for (long j = 0; j <= i; ++j)                                  \
                            acc += row[j] * v[j * W + e];                              \
                        y[at3(b, i, h * d + e, T, C)] = acc / l;                       \
                    }                                                                  \
                    lse[at3(b, i, h, T, H)] = m + LOGF(l);                             \
                }                                                                      \
            }                                                                          \
        free(row);                                                                     \
    }

#define ORACLE_BACKWARD(NAME, REAL, EXPF, SQRTF)                                       \
    void NAME(REAL *grad_x, REAL *D, const REAL *lse, const REAL *grad_y,              \
              const REAL *y, const REAL *qkv, int B, int T, int C, int H)              \
    {                                                                                  \
        const long d = C / H;                                                          \
        const long W = 3L * C;                                                         \
        const REAL scale = (REAL)1 / SQRTF((REAL)d);                                   \
        memset(grad_x, 0, (size_t)B * (size_t)T * (size_t)W * sizeof(REAL));           \
        /* D[b,t,h] = sum_e dO * O, summed over e ascending */                         \
        for (long b = 0; b < B; ++b)                                                   \
            for (long t = 0; t < T; ++t)                                               \
                for (long h = 0; h < H; ++h)                                           \
                {                                                                      \
                    REAL acc = 0;                                                      \
                    for (long e = 0; e < d; ++e)                                       \
                    {                                                                  \
                        const long o = at3(b, t, h * d + e, T, C);                     \
                        acc += grad_y[o] * y[o];                                       \
                    }                                                                  \
                    D[at3(b, t, h, T, H)] = acc;                                       \
                }                                                                      \
        for (long b = 0; b < B; ++b)                                                   \
            for (long h = 0; h < H; ++h)                                               \
            {                                                                          \
                const REAL *q = qkv + at3(b, 0, h * d, T, W);                          \
                const REAL *k = qkv + at3(b, 0, C + h * d, T, W);                      \
                const REAL *v = qkv + at3(b, 0, 2L * C + h * d, T, W);                 \
                const REAL *dO = grad_y + at3(b, 0, h * d, T, C);                      \
                REAL *dq = grad_x + at3(b, 0, h * d, T, W);                            \
                REAL *dk = grad_x + at3(b, 0, C + h * d, T, W);                        \
                REAL *dv = grad_x + at3(b, 0, 2L * C + h * d, T, W);                   \
                for (long i = 0; i < T; ++i)                                           \
                {                                                                      \
                    const REAL L = lse[at3(b, i, h, T, H)];                            \
                    const REAL Di = D[at3(b, i, h, T, H)];                             \
                    for (long j = 0; j <= i; ++j)                                      \
                    {                                                                  \
                        REAL s = 0;                                                    \
                        for (long e = 0; e < d; ++e)                                   \
                            s += q[i * W + e] * k[j * W + e];                          \
                        const REAL p = EXPF(s * scale - L);                            \
                        REAL dp = 0;                                                   \
                        for (long e = 0; e < d; ++e)                                   \
                            dp += dO[i * C + e] * v[j * W + e];                        \
                        const REAL ds = p * (dp - Di) * scale;                         \
                        for (long e = 0; e < d; ++e)                                   \
                        {                                                              \
                            dq[i * W + e] += ds * k[j * W + e];                        \
                            dk[j * W + e] += ds * q[i * W + e];                        \
                            dv[j * W + e] += p * dO[i * C + e];                        \
                        }                                                              \
                    }                                                                  \
                }                                                                      \
            }                                                                          \
    }

ORACLE_FORWARD(oracle_attn_forward_f32, float, expf, logf, sqrtf, -FLT_MAX)
ORACLE_BACKWARD(oracle_attn_backward_f32, float, expf, sqrtf)
ORACLE_FORWARD(oracle_attn_forward_f64, double, exp, log, sqrt, -DBL_MAX)
ORACLE_BACKWARD(oracle_attn_backward_f64, double, exp, sqrt)
