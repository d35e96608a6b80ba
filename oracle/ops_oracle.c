/*
 * ops_oracle.c - CPU restatement of the reference CPU backend's GPT-2 ops
 * around attention. TEST INFRASTRUCTURE ONLY (the checker of
 * gpt_amd/libgpt_hip_ops.so; only tests, smoke() and bench.py's CPU baseline
 * may call it).
 *
 * Each function follows the cited reference function's arithmetic and, for
 * every output element, its accumulation order (which is what makes the
 * results bit-identical to the reference under the same flags); loops that
 * only reorder independent elements are arranged for plain row-major
 * streaming here. Build: oracle/Makefile (-O2 -ffp-contract=off).
 */
#include "ops_oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>

/* cpu_backend.cpp:65-79 */
void ops_oracle_embedding_forward(float *y, const float *wte, const float *wpe, const int *tok, int B, int T, int C)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        const float *e = wte + (long)tok[r] * C, *p = wpe + (r % T) * C;
        float *o = y + r * C;
        for (int h = 0; h < C; ++h)
            o[h] = e[h] + p[h];
    }
}

/* cpu_backend.cpp:81-100: y[r, v] = sum over h ascending of x[r, h] wte[v, h] */
void ops_oracle_unembedding_forward(float *y, const float *x, const float *wte, int B, int T, int C, int Vp)
{
    for (long r = 0; r < (long)B * T; ++r)
        for (int v = 0; v < Vp; ++v)
        {
            const float *a = x + r * C, *e = wte + (long)v * C;
            float s = 0.0f;
            for (int h = 0; h < C; ++h)
                s += a[h] * e[h];
            y[r * Vp + v] = s;
        }
}

/* cpu_backend.cpp:102-117: both tables accumulate over rows in row order */
void ops_oracle_embedding_backward(float *gwte, float *gwpe, const float *gy, const int *tok, int B, int T, int C)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        float *e = gwte + (long)tok[r] * C, *p = gwpe + (r % T) * C;
        const float *g = gy + r * C;
        for (int h = 0; h < C; ++h)
        {
            e[h] += g[h];
            p[h] += g[h];
        }
    }
}

/* cpu_backend.cpp:119-140: grad_x[r, h] = sum over v ascending of
 * gy[r, v] wte[v, h]; grad_wte[v, h] += gy[r, v] x[r, h] over rows in order */
void ops_oracle_unembedding_backward(float *gx, float *gwte, const float *gy, const float *x, const float *wte,
                                     int B, int T, int C, int Vp)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        const float *g = gy + r * Vp, *a = x + r * C;
        for (int h = 0; h < C; ++h)
        {
            float s = 0.0f;
            for (int v = 0; v < Vp; ++v)
            {
                s += g[v] * wte[(long)v * C + h];
                gwte[(long)v * C + h] += g[v] * a[h];
            }
            gx[r * C + h] = s;
        }
    }
}

/* cpu_backend.cpp:142-175 */
void ops_oracle_layernorm_forward(float *y, float *means, float *vars, float *x, const float *res,
                                  const float *gamma, const float *beta, int B, int T, int C)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        float *a = x + r * C;
        float mean = 0.0f, var = 0.0f;
        for (int h = 0; h < C; ++h)
        {
            a[h] += res ? res[r * C + h] : 0.0f;
            mean += a[h];
        }
        mean /= C;
        for (int h = 0; h < C; ++h)
        {
            const float d = a[h] - mean;
            var += d * d;
        }
        var /= C;
        means[r] = mean;
        vars[r] = var;
        for (int h = 0; h < C; ++h)
            y[r * C + h] = ((a[h] - mean) / sqrtf(var + 1e-5f)) * gamma[h] + beta[h];
    }
}

/* cpu_backend.cpp:177-211 */
void ops_oracle_layernorm_backward(float *gx, float *ggamma, float *gbeta, const float *gy, const float *gres,
                                   const float *x, const float *means, const float *vars, const float *gamma, int B,
                                   int T, int C)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        const float *g = gy + r * C, *a = x + r * C;
        const float mean = means[r];
        const float inv_std = 1.0f / sqrtf(vars[r] + 1e-5f);
        float s1 = 0.0f, s2 = 0.0f;
        for (int h = 0; h < C; ++h)
        {
            const float xh = (a[h] - mean) * inv_std;
            ggamma[h] += g[h] * xh;
            gbeta[h] += g[h];
            s1 += g[h] * gamma[h];
            s2 += g[h] * gamma[h] * xh;
        }
        for (int h = 0; h < C; ++h)
        {
            const float xh = (a[h] - mean) * inv_std;
            float o = inv_std * (g[h] * gamma[h] - (s1 / C) - xh * (s2 / C));
            o += gres ? gres[r * C + h] : 0.0f;
            gx[r * C + h] = o;
        }
    }
}

static float gelu_tanh(float s) { return 0.5f * s * (1.0f + tanhf(0.79788456f * (s + 0.044715f * s * s * s))); }

/* cpu_backend.cpp:213-239: the dot product over the input in order, then + b */
void ops_oracle_linear_forward(float *y, float *act, const float *x, const float *w, const float *b, int activation,
                               int B, int T, int in, int out)
{
    for (long r = 0; r < (long)B * T; ++r)
        for (int o = 0; o < out; ++o)
        {
            float s = 0.0f;
            for (int i = 0; i < in; ++i)
                s += x[r * in + i] * w[(long)i * out + o];
            s += b[o];
            y[r * out + o] = s;
            if (activation)
                act[r * out + o] = gelu_tanh(s);
        }
}

/* cpu_backend.cpp:241-266: per row, grad_x starts at 0 and adds over outputs
 * in order; grad_w and grad_b add over rows in order */
void ops_oracle_linear_backward(float *gx, float *gw, float *gb, const float *gy, const float *x, const float *w,
                                int B, int T, int in, int out)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        float *d = gx + r * in;
        memset(d, 0, sizeof(float) * (size_t)in);
        for (int o = 0; o < out; ++o)
        {
            const float g = gy[r * out + o];
            for (int i = 0; i < in; ++i)
            {
                d[i] += g * w[(long)i * out + o];
                gw[(long)i * out + o] += x[r * in + i] * g;
            }
            gb[o] += g;
        }
    }
}

/* cpu_backend.cpp:268-287 */
void ops_oracle_activation_backward(float *gx, const float *gy, const float *x, int B, int T, int n)
{
    for (long k = 0; k < (long)B * T * n; ++k)
    {
        const float v = x[k];
        const float th = tanhf(0.79788456f * (v + 0.044715f * v * v * v));
        const float d = 0.5f * (1.0f + th) + 0.5f * v * (1.0f - th * th) * (0.79788456f + 0.107032f * v * v);
        gx[k] = gy[k] * d;
    }
}

/* cpu_backend.cpp:439-478 */
void ops_oracle_softmax_forward(float *y, const float *x, int B, int T, int V, int Vp)
{
    for (long r = 0; r < (long)B * T; ++r)
    {
        const float *a = x + r * Vp;
        float *o = y + r * Vp;
        float mx = -FLT_MAX;
        for (int v = 0; v < V; ++v)
            if (a[v] > mx)
                mx = a[v];
        float s = 0.0f;
        for (int v = 0; v < V; ++v)
        {
            o[v] = expf(a[v] - mx);
            s += o[v];
        }
        for (int v = 0; v < V; ++v)
            o[v] /= s;
        for (int v = V; v < Vp; ++v)
            o[v] = 0.0f;
    }
}

/* cpu_backend.cpp:480-497 */
void ops_oracle_ce_backward(float *gx, const float *y, const int *labels, int B, int T, int V, int Vp)
{
    const float n = (float)(B * T);
    for (long r = 0; r < (long)B * T; ++r)
        for (int v = 0; v < V; ++v)
            gx[r * Vp + v] = (y[r * Vp + v] - (v == labels[r] ? 1.0f : 0.0f)) / n;
}

/* cpu_backend.cpp:499-515 */
void ops_oracle_ce_loss(float *loss, const float *y, const int *labels, int B, int T, int Vp)
{
    float l = 0.0f;
    for (long r = 0; r < (long)B * T; ++r)
        l -= logf(y[r * Vp + labels[r]] + 1e-8f);
    *loss = l / (float)(B * T);
}

/* cpu_backend.cpp:517-532 */
void ops_oracle_adamw(float *p, const float *g, float *m, float *v, int n, float lr, float beta1, float beta2,
                      float eps, float wd, int step)
{
    const float b1p = powf(beta1, step), b2p = powf(beta2, step);
    for (int i = 0; i < n; ++i)
    {
        m[i] = beta1 * m[i] + (1.0f - beta1) * g[i];
        v[i] = beta2 * v[i] + (1.0f - beta2) * g[i] * g[i];
        const float mh = m[i] / (1.0f - b1p), vh = v[i] / (1.0f - b2p);
        p[i] -= lr * (mh / (sqrtf(vh) + eps) + wd * p[i]);
    }
}

/* cpu_backend.cpp:534-557 */
void ops_oracle_scale_clip(float *g, int n, float max_norm, int accum)
{
    float s = 0.0f;
    for (int i = 0; i < n; ++i)
    {
        g[i] /= accum;
        s += g[i] * g[i];
    }
    const float norm = sqrtf(s);
    if (norm <= max_norm)
        return;
    const float k = max_norm / (norm + 1e-6f);
    for (int i = 0; i < n; ++i)
        g[i] *= k;
}
