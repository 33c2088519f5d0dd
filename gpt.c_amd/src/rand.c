/*
 * Mersenne Twister MT19937 (Matsumoto & Nishimura, 1998) and torch's CPU
 * normal_ transform, written from the published algorithm.
 *
 * Follows the behaviour of /root/reference/include/rand.h:98-221 (which
 * states it is numerically identical to torch): a 624-word state seeded by
 * the Knuth multiplier 1812433253, the standard tempering, floats built
 * from the low 24 bits and doubles from the low 53 bits of the output, and
 * normal values made 16 at a time with Box-Muller (u1 = 1 - x[i],
 * u2 = x[i+8]).  A tail shorter than 16 re-draws the last 16 positions.
 */
#include <math.h>
#include <stdlib.h>
#include "rand.h"

#define MT_UPPER 0x80000000u
#define MT_LOWER 0x7fffffffu
#define MT_TWIST 0x9908b0dfu
#define BM_EPS   1e-12f

void manual_seed(mt19937_state *s, unsigned int seed) {
    s->seed_ = seed;
    s->MATRIX_A[0] = 0u;
    s->MATRIX_A[1] = MT_TWIST;
    s->state_[0] = seed;
    for (unsigned int i = 1; i < MERSENNE_STATE_N; ++i) {
        unsigned int prev = s->state_[i - 1];
        s->state_[i] = 1812433253u * (prev ^ (prev >> 30)) + i;
    }
    s->left_ = 1;
    s->next_ = 0;
}

/* Regenerate all 624 words in place (the "twist"). */
static void mt_twist(mt19937_state *s) {
    unsigned int *st = s->state_;
    for (unsigned int i = 0; i < MERSENNE_STATE_N; ++i) {
        unsigned int nxt = st[(i + 1) % MERSENNE_STATE_N];
        unsigned int y = (st[i] & MT_UPPER) | (nxt & MT_LOWER);
        unsigned int src = st[(i + MERSENNE_STATE_M) % MERSENNE_STATE_N];
        st[i] = src ^ (y >> 1) ^ ((y & 1u) ? MT_TWIST : 0u);
    }
    s->left_ = MERSENNE_STATE_N;
    s->next_ = 0;
}

unsigned int randint32(mt19937_state *s) {
    if (!s) return 0;
    if (s->MATRIX_A[0] != 0u || s->MATRIX_A[1] != MT_TWIST) manual_seed(s, 5489u);
    if (--s->left_ <= 0) mt_twist(s);
    unsigned int y = s->state_[s->next_++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9d2c5680u;
    y ^= (y << 15) & 0xefc60000u;
    y ^= y >> 18;
    return y;
}

unsigned long long randint64(mt19937_state *s) {
    unsigned long long hi = randint32(s);
    unsigned long long lo = randint32(s);
    return (hi << 32) | lo;
}

float randfloat32(mt19937_state *s) {
    return (float)(randint32(s) & 0xffffffu) * (1.0f / 16777216.0f);
}

double randfloat64(mt19937_state *s) {
    return (double)(randint64(s) & ((1ull << 53) - 1)) * (1.0 / 9007199254740992.0);
}

void uniform_(float *data, unsigned int numel, float from, float to, mt19937_state *s) {
    for (unsigned int i = 0; i < numel; ++i) data[i] = randfloat32(s) * (to - from) + from;
}

/* Turn 16 uniforms in x[0..16) into 16 normals: pair (x[i], x[i+8]). */
static void box_muller16(float *x, float mean, float std) {
    for (int i = 0; i < 8; ++i) {
        float r = sqrtf(-2.0f * logf(1.0f - x[i] + BM_EPS));
        float th = (float)(2.0 * M_PI * x[i + 8]);
        x[i] = r * cosf(th) * std + mean;
        x[i + 8] = r * sinf(th) * std + mean;
    }
}

void normal_(float *data, unsigned int numel, float mean, float std, mt19937_state *s) {
    if (numel >= 16) {
        for (unsigned int i = 0; i < numel; ++i) data[i] = randfloat32(s);
        for (unsigned int i = 0; i + 16 <= numel; i += 16) box_muller16(data + i, mean, std);
        if (numel % 16 != 0) {
            float *tail = data + numel - 16;
            for (int i = 0; i < 16; ++i) tail[i] = randfloat32(s);
            box_muller16(tail, mean, std);
        }
        return;
    }
    /* Short tensors: one double-precision pair per two outputs. */
    int have_spare = 0;
    double spare = 0.0;
    for (unsigned int i = 0; i < numel; ++i) {
        if (have_spare) {
            data[i] = (float)(spare * std + mean);
            have_spare = 0;
            continue;
        }
        float u1 = (float)randfloat64(s);
        float u2 = (float)randfloat64(s);
        float r = sqrtf(-2.0f * logf(1.0f - u2 + BM_EPS));
        float th = (float)(2.0 * M_PI * u1);
        spare = r * sinf(th);
        have_spare = 1;
        data[i] = r * cosf(th) * std + mean;
    }
}

void gptc_normal_seeded(float *data, unsigned int numel, float mean, float std, unsigned int seed) {
    mt19937_state *s = (mt19937_state *)malloc(sizeof(mt19937_state));
    if (!s) abort();
    manual_seed(s, seed);
    normal_(data, numel, mean, std, s);
    free(s);
}
