/*
 * TEST INFRASTRUCTURE -- the CPU oracle for the other layers of gpt.c's
 * GPT-2 (Linear, LayerNorm, GELU, Softmax, Embedding, CrossEntropy, AdamW).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; nothing in the product links or calls it.
 *
 * Each function restates one of gpt.c's CPU kernels step for step, on plain
 * arrays instead of tensor_t (the loops, operation order and BLAS calls of
 * the cited lines), so its outputs are what gpt.c's CPU path computes:
 *   linear       kernels/src/cpu/Linear.c:4-80       (OpenBLAS sgemm)
 *   layer norm   kernels/src/cpu/LayerNorm.c:5-124
 *   gelu         kernels/src/cpu/GeLU.c:7-42
 *   softmax      kernels/src/cpu/Softmax.c:7-63
 *   embedding    kernels/src/cpu/Embedding.c:3-47
 *   cross-entr.  kernels/src/cpu/CrossEntropyLoss.c:7-97
 *   adamw        kernels/src/cpu/AdamW.c:5-58
 * gpt.c compiles these with -O3 -march=native -fopenmp; the OpenMP loops
 * are over independent rows, so a serial restatement gives the same values.
 */
#include <math.h>
#include <stddef.h>
#include <stdlib.h>

enum { kNoTrans = 111, kTrans = 112 };

void oracle_sgemm(int ta, int tb, int M, int N, int K, float alpha, const float *A, int lda, const float *Bm, int ldb,
                  float beta, float *Cm, int ldc);

/* y = x W^T (+ b): one sgemm (RowMajor, NoTrans, Trans), then the bias loop. */
void oracle_linear_forward(const float *W, const float *b, const float *x, int rows, int in_f, int out_f, float *y) {
    oracle_sgemm(kNoTrans, kTrans, rows, out_f, in_f, 1.0f, x, in_f, W, in_f, 0.0f, y, out_f);
    if (b != NULL)
        for (int i = 0; i < rows; i++)
            for (int j = 0; j < out_f; j++) y[(size_t)i * out_f + j] += b[j];
}

/* dx = g W (beta 0), dW += g^T x (beta 1), db += sum over rows of g. */
void oracle_linear_backward(const float *g, const float *x, const float *W, int rows, int in_f, int out_f, float *dW,
                            float *db, float *dx) {
    oracle_sgemm(kNoTrans, kNoTrans, rows, in_f, out_f, 1.0f, g, out_f, W, in_f, 0.0f, dx, in_f);
    oracle_sgemm(kTrans, kNoTrans, out_f, in_f, rows, 1.0f, g, out_f, x, in_f, 1.0f, dW, in_f);
    if (db != NULL)
        for (int i = 0; i < rows; i++)
            for (int j = 0; j < out_f; j++) db[j] += g[(size_t)i * out_f + j];
}

/* One pass of sum and sum of squares per row; var = E[x^2] - mean^2. */
void oracle_layer_norm_forward(const float *x, const float *W, const float *b, int rows, int C, float eps,
                               float *mean, float *rstd, float *y) {
    const float scale = 1.0f / C;
    for (int i = 0; i < rows; i++) {
        const float *xr = x + (size_t)i * C;
        float *yr = y + (size_t)i * C;
        float s = 0.0f, ss = 0.0f;
        for (int j = 0; j < C; j++) {
            s += xr[j];
            ss += xr[j] * xr[j];
        }
        const float m = s * scale;
        const float nb = -m;
        const float var = ss * scale - m * m;
        const float r = 1.0f / sqrtf(var + eps);
        for (int j = 0; j < C; j++) yr[j] = (xr[j] + nb) * r * W[j] + (b ? b[j] : 0.0f);
        mean[i] = m;
        rstd[i] = r;
    }
}

/* dW += g (a x + b), db += g, dx += a g W + b' x + c' (accumulating). */
void oracle_layer_norm_backward(const float *g, const float *x, const float *mean, const float *rstd, const float *W,
                                int rows, int C, float *dW, float *db, float *dx) {
    const float scale = 1.0f / C;
    for (int i = 0; i < rows; i++) {
        const float *xr = x + (size_t)i * C;
        const float *gr = g + (size_t)i * C;
        float *dr = dx + (size_t)i * C;
        {
            const float a = rstd[i];
            const float bb = -a * mean[i];
            for (int j = 0; j < C; j++) dW[j] += gr[j] * (a * xr[j] + bb);
        }
        if (db)
            for (int j = 0; j < C; j++) db[j] += gr[j];
        float ds = 0.0f, dbs = 0.0f;
        for (int j = 0; j < C; j++) {
            ds += gr[j] * xr[j] * W[j];
            dbs += gr[j] * W[j];
        }
        const float a = rstd[i];
        const float bb = (dbs * mean[i] - ds) * a * a * a * scale;
        const float c = -bb * mean[i] - dbs * a * scale;
        for (int j = 0; j < C; j++) dr[j] += a * gr[j] * W[j] + bb * xr[j] + c;
    }
}

/* sqrt(2) * (2/sqrt(pi)) * 0.5 evaluated in double, then used as float. */
static const float kBeta = (float)(M_SQRT2 * M_2_SQRTPI * 0.5);

void oracle_gelu_forward(const float *x, long n, float *y) {
    for (long i = 0; i < n; i++) {
        const float xi = x[i];
        const float cube = 0.044715f * xi * xi * xi;
        y[i] = 0.5f * xi * (1.0f + tanhf(kBeta * (xi + cube)));
    }
}

void oracle_gelu_backward(const float *g, const float *x, long n, float *dx) {
    for (long i = 0; i < n; i++) {
        const float xi = x[i];
        const float sq = xi * xi;
        const float cube = sq * xi;
        const float inner = kBeta * (xi + 0.044715f * cube);
        const float th = tanhf(inner);
        const float left = 0.5f * xi;
        const float right = 1.0f + th;
        const float left_d = 0.5f * right;
        const float tanh_d = 1.0f - th * th;
        const float inner_d = kBeta * (1.0f + 3.0f * 0.044715f * sq);
        const float right_d = left * tanh_d * inner_d;
        dx[i] = g[i] * (left_d + right_d);
    }
}

/* max, then exp and sum, then a reciprocal multiply. */
void oracle_softmax_forward(const float *x, int rows, int C, float *y) {
    for (int i = 0; i < rows; i++) {
        const float *xr = x + (size_t)i * C;
        float *yr = y + (size_t)i * C;
        float mx = -INFINITY;
        for (int j = 0; j < C; j++) mx = fmaxf(mx, xr[j]);
        float sum = 0.0f;
        for (int j = 0; j < C; j++) {
            const float e = expf(xr[j] - mx);
            sum += e;
            yr[j] = e;
        }
        sum = 1.0f / sum;
        for (int j = 0; j < C; j++) yr[j] = yr[j] * sum;
    }
}

void oracle_softmax_backward(const float *g, const float *p, int rows, int C, float *dx) {
    for (int i = 0; i < rows; i++) {
        const float *gr = g + (size_t)i * C;
        const float *pr = p + (size_t)i * C;
        float *dr = dx + (size_t)i * C;
        float sum = 0.0f;
        for (int j = 0; j < C; j++) sum += gr[j] * pr[j];
        for (int j = 0; j < C; j++) dr[j] = (gr[j] - sum) * pr[j];
    }
}

void oracle_embedding_forward(const float *W, const float *ids, int rows, int C, float *y) {
    for (int i = 0; i < rows; i++) {
        const float *w = W + (size_t)(int)ids[i] * C;
        for (int j = 0; j < C; j++) y[(size_t)i * C + j] = w[j];
    }
}

/* dW[ids[i % L]] += g[i] in row order. */
void oracle_embedding_backward(const float *g, const float *ids, int rows, int L, int C, float *dW) {
    for (int i = 0; i < rows; i++) {
        float *w = dW + (size_t)(int)ids[i % L] * C;
        for (int j = 0; j < C; j++) w[j] += g[(size_t)i * C + j];
    }
}

/* lsm = x - max - log(sum exp(x - max)); loss = mean of -lsm[target]. */
void oracle_cross_entropy_forward(const float *logits, const float *targets, int rows, int V, float *lsm,
                                  float *loss) {
    float *per = (float *)malloc(sizeof(float) * (size_t)(rows > 0 ? rows : 1));
    for (int i = 0; i < rows; i++) {
        const float *xr = logits + (size_t)i * V;
        float *lr = lsm + (size_t)i * V;
        float mx = -INFINITY;
        for (int j = 0; j < V; j++) mx = fmaxf(mx, xr[j]);
        float sum = 0.0f;
        for (int j = 0; j < V; j++) sum += expf(xr[j] - mx);
        sum = logf(sum);
        for (int j = 0; j < V; j++) lr[j] = xr[j] - mx - sum;
        per[i] = -lr[(int)targets[i]];
    }
    float total = 0.0f;
    for (int i = 0; i < rows; i++) total += per[i];
    *loss = total / rows;
    free(per);
}

/* dx starts at zero (the layer zeroes it, src/loss.c:73-108); the target
 * entry gets -g/(B T), then dx = dlsm - exp(lsm) * sum(dlsm). */
void oracle_cross_entropy_backward(const float *g, const float *lsm, const float *targets, int rows, int V,
                                   float *dx) {
    const int bt = rows;
    for (size_t i = 0; i < (size_t)rows * V; i++) dx[i] = 0.0f;
    for (int i = 0; i < rows; i++) dx[(size_t)i * V + (int)targets[i]] = -g[i] / bt;
    for (int i = 0; i < rows; i++) {
        const float *lr = lsm + (size_t)i * V;
        float *dr = dx + (size_t)i * V;
        float sum = 0.0f;
        for (int j = 0; j < V; j++) sum += dr[j];
        for (int j = 0; j < V; j++) dr[j] = dr[j] - expf(lr[j]) * sum;
    }
}

static inline float lerpf_ref(float start, float end, float weight) {
    return fmaf(weight, end, fmaf(-weight, start, start));
}

void oracle_adamw(float *p, const float *g, float *m, float *v, long n, float lr, float beta1, float beta2,
                  float weight_decay, float eps, int step) {
    const float c1 = 1.0f - powf(beta1, step);
    const float c2 = 1.0f - powf(beta2, step);
    for (long j = 0; j < n; j++) {
        p[j] -= lr * weight_decay * p[j];
        const float mn = lerpf_ref(g[j], m[j], beta1);
        const float vn = lerpf_ref(g[j] * g[j], v[j], beta2);
        const float m_hat = mn / c1;
        const float v_hat = vn / c2;
        m[j] = mn;
        v[j] = vn;
        p[j] -= lr * m_hat / (sqrtf(v_hat) + eps);
    }
}
