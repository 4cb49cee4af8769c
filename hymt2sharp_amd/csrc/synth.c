/*
 * synth.c -- seeded synthetic inputs for tests and benchmarks.
 *
 * xoshiro256** seeded through SplitMix64, the construction of the
 * reference's sampler RNG (Sampling.cs:375-409); uniform floats are
 * (next >> 40) * 2^-24 as NextSingle; normals are Box-Muller in fp64.
 */
#include <math.h>
#include <stdint.h>

typedef struct {
    uint64_t s[4];
} xoshiro;

static uint64_t splitmix(uint64_t *z)
{
    *z += 0x9E3779B97F4A7C15ULL;
    uint64_t x = *z;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

static inline uint64_t rotl(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

static void seed(xoshiro *r, uint64_t s)
{
    for (int i = 0; i < 4; i++) r->s[i] = splitmix(&s);
}

static uint64_t next(xoshiro *r)
{
    uint64_t *s = r->s;
    uint64_t out = rotl(s[1] * 5, 7) * 9;
    uint64_t t = s[1] << 17;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = rotl(s[3], 45);
    return out;
}

static double uniform01(xoshiro *r) { return (double)(next(r) >> 40) * (1.0 / 16777216.0); }

/* out[i] = lo + (hi - lo) * U[0,1) */
void hymt_synth_uniform(uint64_t s, float *out, long n, float lo, float hi)
{
    xoshiro r;
    seed(&r, s);
    for (long i = 0; i < n; i++) out[i] = (float)(lo + (hi - lo) * uniform01(&r));
}

/* out[i] = scale * N(0,1), Box-Muller pairs */
void hymt_synth_normal(uint64_t s, float *out, long n, float scale)
{
    xoshiro r;
    seed(&r, s);
    const double two_pi = 6.283185307179586476925286766559;
    for (long i = 0; i < n; i += 2) {
        double u1 = 1.0 - uniform01(&r); /* (0, 1] */
        double u2 = uniform01(&r);
        double rad = sqrt(-2.0 * log(u1));
        out[i] = (float)(scale * rad * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(scale * rad * sin(two_pi * u2));
    }
}

/* out[i] = next() % modulus */
void hymt_synth_index(uint64_t s, int64_t *out, long n, int64_t modulus)
{
    xoshiro r;
    seed(&r, s);
    for (long i = 0; i < n; i++) out[i] = (int64_t)(next(&r) % (uint64_t)modulus);
}
