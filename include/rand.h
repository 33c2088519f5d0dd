/*
 * rand.h -- seeded input generator, numerically identical to torch's CPU
 * generator (mt19937 + the Box-Muller `normal_` transform).
 *
 * Same API and state layout as /root/reference/include/rand.h:96-221, so
 * inputs drawn here match gpt.c's tooling and `torch.manual_seed(s);
 * torch.empty(n).normal_()` bit for bit.  The algorithm is the public
 * Mersenne Twister of Matsumoto & Nishimura (1998) plus torch's normal
 * transform (groups of 16 uniforms -> 8 cos/sin pairs; fewer than 16
 * values drawn from double uniforms).  Implemented in gpt.c_amd/src/rand.c.
 */
#pragma once

#ifdef __cplusplus
extern "C" {
#endif

#define MERSENNE_STATE_M 397u
#define MERSENNE_STATE_N 624u

typedef struct {
    unsigned long long seed_;
    int left_;
    unsigned int next_;
    unsigned int state_[MERSENNE_STATE_N];
    unsigned int MATRIX_A[2];
} mt19937_state;

void manual_seed(mt19937_state *state, unsigned int seed);
unsigned int randint32(mt19937_state *state);
unsigned long long randint64(mt19937_state *state);
float randfloat32(mt19937_state *state);
double randfloat64(mt19937_state *state);
void uniform_(float *data, unsigned int numel, float from, float to, mt19937_state *state);
void normal_(float *data, unsigned int numel, float mean, float std, mt19937_state *state);

/* Convenience for callers without the struct layout (Python/ctypes):
 * fill data[0..numel) with normal_(mean, std) drawn from a fresh
 * manual_seed(seed) state. */
void gptc_normal_seeded(float *data, unsigned int numel, float mean, float std, unsigned int seed);

#ifdef __cplusplus
}
#endif
