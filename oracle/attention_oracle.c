/*
 * TEST INFRASTRUCTURE -- the CPU oracle for the causal attention path.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker or the timed CPU baseline.  Nothing in
 * the product (gpt.c_amd/) links or calls it.
 *
 * A C restatement of gpt.c's CPU attention kernel,
 * /root/reference/kernels/src/cpu/Attention.c:8-301, step for step:
 *   forward  (:46-167)  permute qkv (B,T,3C) -> q,k,v (B,H,T,D) (:99-122);
 *                       per head S = (1/sqrt(D)) Q K^T with one
 *                       cblas_sgemm(RowMajor, NoTrans, Trans, T,T,D, alpha)
 *                       (:125-133); -inf where mask != 1 (:135-142);
 *                       row softmax with max subtraction, expf and a
 *                       reciprocal multiply (:8-29,144); per head O = P V
 *                       with cblas_sgemm(NoTrans, NoTrans, T,D,T) (:147-156);
 *                       unpermute to (B,T,C) (:158-164).  att keeps P.
 *   backward (:169-301) unpermute dO (:203-209); per head dP = dO V^T and
 *                       dV = P^T dO (:212-241); dS = (dP - rowsum(dP*P))*P
 *                       (:31-44,243); dQ = alpha dS K and dK = alpha dS^T Q
 *                       (:245-275); scatter into dqkv (B,T,3C) (:277-297).
 * The reference reuses buffers (permuted dO in dout, dQ in global_grad, dK
 * in the v cache, :198-201); the values are the same, so this restatement
 * uses separate scratch instead and leaves its inputs intact.
 *
 * BLAS: the full-T^2 single-precision GEMMs run on OpenBLAS loaded at run
 * time with dlopen (the OpenBLAS shipped in the scipy/numpy wheels of this
 * image; LP64 "scipy_cblas_sgemm" preferred, ILP64 "..64_" accepted).
 * There is no naive-loop substitute: without OpenBLAS, oracle_init fails.
 * Also here: the fp64 brute-force reference used to pin the above.
 */
#include <dlfcn.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* CBLAS enumerators (values fixed by the CBLAS interface). */
enum { kRowMajor = 101, kNoTrans = 111, kTrans = 112 };

typedef void (*sgemm32_fn)(int, int, int, int, int, int, float, const float *, int, const float *, int, float,
                           float *, int);
typedef void (*sgemm64_fn)(int, int, int, int64_t, int64_t, int64_t, float, const float *, int64_t, const float *,
                           int64_t, float, float *, int64_t);
typedef char *(*config_fn)(void);
typedef void (*threads32_fn)(int);
typedef void (*threads64_fn)(int64_t);

static void *g_lib;
static sgemm32_fn g_sgemm32;
static sgemm64_fn g_sgemm64;
static config_fn g_config;
static threads32_fn g_threads32;
static threads64_fn g_threads64;
static char g_path[1024];

static void *sym(const char *a, const char *b) {
    void *p = dlsym(g_lib, a);
    if (!p && b) p = dlsym(g_lib, b);
    return p;
}

/* Load OpenBLAS from `path`.  Returns 0 on success, -1 (with a message on
 * stderr) when the library or its sgemm entry point is missing. */
int oracle_init(const char *path) {
    if (g_lib) return 0;
    if (!path || !*path) {
        fprintf(stderr, "[oracle] no OpenBLAS path given\n");
        return -1;
    }
    g_lib = dlopen(path, RTLD_NOW | RTLD_LOCAL);
    if (!g_lib) {
        fprintf(stderr, "[oracle] dlopen(%s) failed: %s\n", path, dlerror());
        return -1;
    }
    g_sgemm32 = (sgemm32_fn)sym("scipy_cblas_sgemm", "cblas_sgemm");
    if (!g_sgemm32) g_sgemm64 = (sgemm64_fn)sym("scipy_cblas_sgemm64_", "cblas_sgemm64_");
    g_config = (config_fn)sym("scipy_openblas_get_config", "openblas_get_config");
    if (!g_config) g_config = (config_fn)sym("scipy_openblas_get_config64_", "openblas_get_config64_");
    g_threads32 = (threads32_fn)sym("scipy_openblas_set_num_threads", "openblas_set_num_threads");
    if (!g_threads32) g_threads64 = (threads64_fn)sym("scipy_openblas_set_num_threads64_", "openblas_set_num_threads64_");
    if (!g_sgemm32 && !g_sgemm64) {
        fprintf(stderr, "[oracle] %s exports no cblas sgemm\n", path);
        dlclose(g_lib);
        g_lib = NULL;
        return -1;
    }
    snprintf(g_path, sizeof g_path, "%s", path);
    return 0;
}

const char *oracle_blas_config(void) {
    static char buf[1400];
    snprintf(buf, sizeof buf, "%s [%s, %s]", g_config ? g_config() : "unknown", g_path,
             g_sgemm32 ? "LP64" : "ILP64");
    return buf;
}

void oracle_set_threads(int n) {
    if (g_threads32) g_threads32(n);
    else if (g_threads64) g_threads64(n);
}

/* Row-major cblas_sgemm through the loaded OpenBLAS (ta/tb: kNoTrans or
 * kTrans); also used by ops_oracle.c. */
void oracle_sgemm(int ta, int tb, int M, int N, int K, float alpha, const float *A, int lda, const float *Bm, int ldb,
                  float beta, float *Cm, int ldc) {
    if (!g_lib) {
        fprintf(stderr, "[oracle] oracle_init was not called\n");
        abort();
    }
    if (g_sgemm32)
        g_sgemm32(kRowMajor, ta, tb, M, N, K, alpha, A, lda, Bm, ldb, beta, Cm, ldc);
    else
        g_sgemm64(kRowMajor, ta, tb, M, N, K, alpha, A, lda, Bm, ldb, beta, Cm, ldc);
}

/* Row softmax in place (cpu/Attention.c:8-29). */
static void softmax_rows(float *x, long rows, int n) {
    for (long i = 0; i < rows; i++) {
        float *r = x + i * (long)n;
        float mx = -INFINITY;
        for (int j = 0; j < n; j++) mx = fmaxf(mx, r[j]);
        float sum = 0.0f;
        for (int j = 0; j < n; j++) {
            float e = expf(r[j] - mx);
            sum += e;
            r[j] = e;
        }
        float inv = 1.0f / sum;
        for (int j = 0; j < n; j++) r[j] *= inv;
    }
}

/* dx = (g - rowsum(g * p)) * p, written over g (cpu/Attention.c:31-44). */
static void softmax_rows_backward(float *g, const float *p, long rows, int n) {
    for (long i = 0; i < rows; i++) {
        float *gr = g + i * (long)n;
        const float *pr = p + i * (long)n;
        float sum = 0.0f;
        for (int j = 0; j < n; j++) sum += gr[j] * pr[j];
        for (int j = 0; j < n; j++) gr[j] = (gr[j] - sum) * pr[j];
    }
}

/*
 * x (B,T,3C) -> out (B,T,C).  q,k,v (B,H,T,D) and att (B,H,T,T) are the
 * reference's caches and are filled here.  mask is (rows >= T) x mask_row,
 * 1.0 where attention is allowed.
 */
void oracle_attention_forward(const float *x, int B, int T, int C, int H, const float *mask, int mask_row, float *q,
                              float *k, float *v, float *att, float *out) {
    const int D = C / H, C3 = 3 * C;
    const float scale = 1.0f / sqrtf((float)D);
    const long TD = (long)T * D, TT = (long)T * T;

    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++)
            for (int t = 0; t < T; t++) {
                const float *row = x + ((long)b * T + t) * C3 + (long)h * D;
                const long dst = ((long)b * H + h) * TD + (long)t * D;
                memcpy(q + dst, row, sizeof(float) * D);
                memcpy(k + dst, row + C, sizeof(float) * D);
                memcpy(v + dst, row + 2 * C, sizeof(float) * D);
            }

    for (long i = 0; i < (long)B * H; i++)
        oracle_sgemm(kNoTrans, kTrans, T, T, D, scale, q + i * TD, D, k + i * TD, D, 0.0f, att + i * TT, T);

    for (long i = 0; i < (long)B * H; i++)
        for (int r = 0; r < T; r++) {
            float *ar = att + i * TT + (long)r * T;
            for (int c = 0; c < T; c++)
                if (mask[(long)r * mask_row + c] != 1.0f) ar[c] = -INFINITY;
        }

    softmax_rows(att, (long)B * H * T, T);

    float *o = (float *)malloc(sizeof(float) * (size_t)B * H * TD + 64);
    if (!o) abort();
    for (long i = 0; i < (long)B * H; i++)
        oracle_sgemm(kNoTrans, kNoTrans, T, D, T, 1.0f, att + i * TT, T, v + i * TD, D, 0.0f, o + i * TD, D);

    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                memcpy(out + ((long)b * T + t) * C + (long)h * D, o + ((long)b * H + h) * TD + (long)t * D,
                       sizeof(float) * D);
    free(o);
}

/*
 * dy (B,T,C) + caches q,k,v (B,H,T,D), att = P (B,H,T,T) -> dqkv (B,T,3C).
 * Inputs are not modified.
 */
void oracle_attention_backward(const float *dy, int B, int T, int C, int H, const float *q, const float *k,
                               const float *v, const float *att, float *dqkv) {
    const int D = C / H, C3 = 3 * C;
    const float scale = 1.0f / sqrtf((float)D);
    const long TD = (long)T * D, TT = (long)T * T, n = (long)B * H * TD;

    float *g = (float *)malloc(sizeof(float) * (size_t)n + 64);
    float *dq = (float *)malloc(sizeof(float) * (size_t)n + 64);
    float *dk = (float *)malloc(sizeof(float) * (size_t)n + 64);
    float *dv = (float *)malloc(sizeof(float) * (size_t)n + 64);
    float *datt = (float *)malloc(sizeof(float) * (size_t)B * H * TT + 64);
    if (!g || !dq || !dk || !dv || !datt) abort();

    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++)
                memcpy(g + ((long)b * H + h) * TD + (long)t * D, dy + ((long)b * T + t) * C + (long)h * D,
                       sizeof(float) * D);

    for (long i = 0; i < (long)B * H; i++) {
        oracle_sgemm(kNoTrans, kTrans, T, T, D, 1.0f, g + i * TD, D, v + i * TD, D, 0.0f, datt + i * TT, T);
        oracle_sgemm(kTrans, kNoTrans, T, D, T, 1.0f, att + i * TT, T, g + i * TD, D, 0.0f, dv + i * TD, D);
    }

    softmax_rows_backward(datt, att, (long)B * H * T, T);

    for (long i = 0; i < (long)B * H; i++) {
        oracle_sgemm(kNoTrans, kNoTrans, T, D, T, scale, datt + i * TT, T, k + i * TD, D, 0.0f, dq + i * TD, D);
        oracle_sgemm(kTrans, kNoTrans, T, D, T, scale, datt + i * TT, T, q + i * TD, D, 0.0f, dk + i * TD, D);
    }

    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++) {
            float *row = dqkv + ((long)b * T + t) * C3;
            for (int h = 0; h < H; h++) {
                const long src = ((long)b * H + h) * TD + (long)t * D;
                memcpy(row + (long)h * D, dq + src, sizeof(float) * D);
                memcpy(row + C + (long)h * D, dk + src, sizeof(float) * D);
                memcpy(row + 2 * C + (long)h * D, dv + src, sizeof(float) * D);
            }
        }
    free(g);
    free(dq);
    free(dk);
    free(dv);
    free(datt);
}

/*
 * fp64 brute force of the same mathematics, one (b, h) at a time, used to
 * pin the restatement above: y (B,T,C), lse (B,H,T) (natural log), and,
 * when dy != NULL, dqkv (B,T,3C).  Causal rule: key j attends to query i
 * iff j <= i.  O(T^2 D) per head with O(T) scratch.
 */
void oracle_attention_fp64(const float *x, const float *dy, int B, int T, int C, int H, double *y, double *lse,
                           double *dqkv) {
    const int D = C / H, C3 = 3 * C;
    const double scale = 1.0 / sqrt((double)D);
    double *p = (double *)malloc(sizeof(double) * (size_t)T + 64);
    double *dp = (double *)malloc(sizeof(double) * (size_t)T + 64);
    if (!p || !dp) abort();
    if (dqkv) memset(dqkv, 0, sizeof(double) * (size_t)B * T * C3);
    for (int b = 0; b < B; b++)
        for (int h = 0; h < H; h++) {
            const float *base = x + (long)b * T * C3 + (long)h * D;
            for (int i = 0; i < T; i++) {
                const float *qi = base + (long)i * C3;
                double mx = -INFINITY;
                for (int j = 0; j <= i; j++) {
                    const float *kj = base + (long)j * C3 + C;
                    double s = 0.0;
                    for (int d = 0; d < D; d++) s += (double)qi[d] * (double)kj[d];
                    p[j] = s * scale;
                    if (p[j] > mx) mx = p[j];
                }
                double sum = 0.0;
                for (int j = 0; j <= i; j++) {
                    p[j] = exp(p[j] - mx);
                    sum += p[j];
                }
                for (int j = 0; j <= i; j++) p[j] /= sum;
                if (lse) lse[((long)b * H + h) * T + i] = mx + log(sum);
                double *yi = y + ((long)b * T + i) * C + (long)h * D;
                for (int d = 0; d < D; d++) {
                    double acc = 0.0;
                    for (int j = 0; j <= i; j++) acc += p[j] * (double)base[(long)j * C3 + 2 * C + d];
                    yi[d] = acc;
                }
                if (!dqkv) continue;
                const float *gi = dy + ((long)b * T + i) * C + (long)h * D;
                double rs = 0.0;
                for (int j = 0; j <= i; j++) {
                    const float *vj = base + (long)j * C3 + 2 * C;
                    double s = 0.0;
                    for (int d = 0; d < D; d++) s += (double)gi[d] * (double)vj[d];
                    dp[j] = s;
                    rs += s * p[j];
                }
                double *dqi = dqkv + ((long)b * T + i) * C3 + (long)h * D;
                for (int j = 0; j <= i; j++) {
                    const double ds = p[j] * (dp[j] - rs) * scale;
                    const float *kj = base + (long)j * C3 + C;
                    double *dkj = dqkv + ((long)b * T + j) * C3 + C + (long)h * D;
                    double *dvj = dqkv + ((long)b * T + j) * C3 + 2 * C + (long)h * D;
                    for (int d = 0; d < D; d++) {
                        dqi[d] += ds * (double)kj[d];
                        dkj[d] += ds * (double)qi[d];
                        dvj[d] += p[j] * (double)gi[d];
                    }
                }
            }
        }
    free(p);
    free(dp);
}
