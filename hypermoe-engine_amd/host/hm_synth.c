/*
 * hm_synth.c -- seeded synthetic inputs for the MoE block (host, C11).
 *
 * The reference has no PRNG (std::normal_distribution is implementation
 * defined), so this build documents its own, reproducible on any IEEE-754
 * host because it uses only +, -, *, / and sqrt (correctly rounded), never
 * libm transcendentals:
 *
 *   mix(z)       = SplitMix64 finaliser:
 *                  z ^= z>>30; z *= 0xBF58476D1CE4E5B9;
 *                  z ^= z>>27; z *= 0x94D049BB133111EB; z ^= z>>31
 *   key(seed,tag)= mix(seed + mix(tag))
 *   out_i        = mix(key + (i+1) * 0x9E3779B97F4A7C15),  i = 0, 1, ...
 *   pair j from out_{2j}, out_{2j+1}:
 *       u1 = ((out_{2j} >> 11) + 1) * 2^-53      in (0, 1]
 *       u2 = (out_{2j+1} >> 11) * 2^-53          in [0, 1)
 *       r  = sqrt(-2 * ln(u1));  z0 = r cos(2 pi u2);  z1 = r sin(2 pi u2)
 *   value_{2j} = (float)(mean + std * z0), value_{2j+1} = (float)(mean + std * z1)
 *
 *   ln(u):  u = m 2^e with m in [sqrt(1/2), sqrt(2)) (exact bit split),
 *           f = (m-1)/(m+1), ln m = 2 f (1 + f^2/3 + ... + f^20/21) (Horner),
 *           ln u = e * LN2 + ln m.
 *   cos/sin(2 pi u): q = floor(4u), theta = (4u - q) * pi/2 in [0, pi/2),
 *           Taylor series to theta^24 / theta^25 (Horner), then the exact
 *           quadrant rotation (c, s) -> (-s, c) -> (-c, -s) -> (s, -c).
 *
 * Tags: hidden states 1; router weights of layer l 0x100 + l; expert weights
 * (layer l, expert e, projection p in {0 gate, 1 up, 2 down}):
 * (1<<40) | (l<<20) | (e<<4) | p.
 * Build: gcc -O3 -ffp-contract=off (no FMA contraction).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define HM_GOLDEN 0x9E3779B97F4A7C15ull
#define HM_LN2 0x1.62e42fefa39efp-1
#define HM_PI_2 0x1.921fb54442d18p+0

static uint64_t mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBull;
    z ^= z >> 31;
    return z;
}

uint64_t hm_synth_key(uint64_t seed, uint64_t tag) { return mix64(seed + mix64(tag)); }

uint64_t hm_synth_u64(uint64_t key, uint64_t index) {
    return mix64(key + (index + 1) * HM_GOLDEN);
}

/* ln(u) for u in (0, 1] with only basic IEEE operations. */
double hm_synth_ln(double u) {
    uint64_t bits;
    memcpy(&bits, &u, sizeof bits);
    int e = (int)((bits >> 52) & 0x7ff) - 1022;  /* u = m * 2^e, m in [0.5, 1) */
    bits = (bits & 0x000fffffffffffffull) | 0x3fe0000000000000ull;
    double m;
    memcpy(&m, &bits, sizeof m);
    if (m < 0x1.6a09e667f3bcdp-1) { /* sqrt(1/2) */
        m = m * 2.0;
        e -= 1;
    }
    const double f = (m - 1.0) / (m + 1.0);
    const double f2 = f * f;
    double p = 1.0 / 21.0;
    p = p * f2 + 1.0 / 19.0;
    p = p * f2 + 1.0 / 17.0;
    p = p * f2 + 1.0 / 15.0;
    p = p * f2 + 1.0 / 13.0;
    p = p * f2 + 1.0 / 11.0;
    p = p * f2 + 1.0 / 9.0;
    p = p * f2 + 1.0 / 7.0;
    p = p * f2 + 1.0 / 5.0;
    p = p * f2 + 1.0 / 3.0;
    p = p * f2 + 1.0;
    return (double)e * HM_LN2 + 2.0 * f * p;
}

/* cos(2 pi u), sin(2 pi u) for u in [0, 1). */
void hm_synth_cossin(double u, double* c_out, double* s_out) {
    const double x = u * 4.0;
    const double qd = floor(x);
    const int q = (int)qd;
    const double th = (x - qd) * HM_PI_2;
    const double t2 = th * th;
    /* 1/(2n)! and 1/(2n+1)!, n = 0..12 (constant-folded, correctly rounded) */
    static const double inv_fact_even[13] = {
        1.0, 1.0 / 2.0, 1.0 / 24.0, 1.0 / 720.0, 1.0 / 40320.0,
        1.0 / 3628800.0, 1.0 / 479001600.0, 1.0 / 87178291200.0,
        1.0 / 20922789888000.0, 1.0 / 6402373705728000.0,
        1.0 / 2432902008176640000.0, 1.0 / 1124000727777607680000.0,
        1.0 / 620448401733239439360000.0};
    static const double inv_fact_odd[13] = {
        1.0, 1.0 / 6.0, 1.0 / 120.0, 1.0 / 5040.0, 1.0 / 362880.0,
        1.0 / 39916800.0, 1.0 / 6227020800.0, 1.0 / 1307674368000.0,
        1.0 / 355687428096000.0, 1.0 / 121645100408832000.0,
        1.0 / 51090942171709440000.0, 1.0 / 25852016738884976640000.0,
        1.0 / 15511210043330985984000000.0};
    /* Horner in -t^2: cos = sum (-1)^n t^(2n)/(2n)!, sin = t sum (-1)^n t^(2n)/(2n+1)! */
    double pc = inv_fact_even[12];
    double ps = inv_fact_odd[12];
    for (int n = 11; n >= 0; --n) {
        pc = pc * (-t2) + inv_fact_even[n];
        ps = ps * (-t2) + inv_fact_odd[n];
    }
    const double c = pc;
    const double s = ps * th;
    switch (q & 3) {
    case 0: *c_out = c; *s_out = s; break;
    case 1: *c_out = -s; *s_out = c; break;
    case 2: *c_out = -c; *s_out = -s; break;
    default: *c_out = s; *s_out = -c; break;
    }
}

/* n normal floats with the given mean/std from stream key(seed, tag). */
void hm_synth_normal(uint64_t seed, uint64_t tag, int64_t n, float mean, float std,
                     float* out) {
    const uint64_t key = hm_synth_key(seed, tag);
    for (int64_t j = 0; 2 * j < n; ++j) {
        const uint64_t a = hm_synth_u64(key, (uint64_t)(2 * j));
        const uint64_t b = hm_synth_u64(key, (uint64_t)(2 * j + 1));
        const double u1 = (double)((a >> 11) + 1) * 0x1p-53;
        const double u2 = (double)(b >> 11) * 0x1p-53;
        const double r = sqrt(-2.0 * hm_synth_ln(u1));
        double c, s;
        hm_synth_cossin(u2, &c, &s);
        out[2 * j] = (float)((double)mean + (double)std * (r * c));
        if (2 * j + 1 < n) out[2 * j + 1] = (float)((double)mean + (double)std * (r * s));
    }
}

/* Reference packer semantics (src/tensor/quantization/Quantization.cpp:45-79). */
static void quantize_int8(const float* w, int64_t n, int8_t* q, float* scale) {
    float maximum = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float m = fabsf(w[i]);
        if (m > maximum) maximum = m;
    }
    const float s = maximum == 0.0f ? 1.0f : maximum / 127.0f;
    for (int64_t i = 0; i < n; ++i) {
        float r = roundf(w[i] / s);
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        q[i] = (int8_t)r;
    }
    *scale = s;
}

typedef struct {
    uint64_t seed, layer;
    int64_t experts, hidden, inter;
    float std;
    int int8;
    void* payload;
    float* scale;
    int32_t* zp;
    int64_t next;
    pthread_mutex_t lock;
} layer_job;

static void* layer_worker(void* arg) {
    layer_job* job = (layer_job*)arg;
    const int64_t H = job->hidden, I = job->inter, per = H * I;
    float* tmp = job->int8 ? (float*)malloc((size_t)per * sizeof(float)) : NULL;
    for (;;) {
        pthread_mutex_lock(&job->lock);
        const int64_t item = job->next++;
        pthread_mutex_unlock(&job->lock);
        if (item >= job->experts * 3) break;
        const int64_t e = item / 3, p = item % 3;
        const uint64_t tag = (1ull << 40) | (job->layer << 20) | ((uint64_t)e << 4) | (uint64_t)p;
        if (job->int8) {
            hm_synth_normal(job->seed, tag, per, 0.0f, job->std, tmp);
            quantize_int8(tmp, per, (int8_t*)job->payload + item * per, &job->scale[item]);
            job->zp[item] = 0;
        } else {
            hm_synth_normal(job->seed, tag, per, 0.0f, job->std,
                            (float*)job->payload + item * per);
        }
    }
    free(tmp);
    return NULL;
}

/* One layer of expert weights in the reference payload layout: expert e =
 * gate [H x I] | up [H x I] | down [I x H] (each ~N(0, std) drawn in row-major
 * order of its INPUT_OUTPUT matrix), INT8-packed per projection when int8 is
 * set (scale/zp [E x 3]).  Uses up to `threads` worker threads; the result
 * does not depend on the thread count. */
int hm_synth_layer(uint64_t seed, uint64_t layer, int64_t experts, int64_t hidden,
                   int64_t inter, float std, int int8, void* payload, float* scale,
                   int32_t* zp, int threads) {
    if (!payload || experts <= 0 || hidden <= 0 || inter <= 0) return 1;
    if (int8 && (!scale || !zp)) return 1;
    layer_job job;
    job.seed = seed; job.layer = layer; job.experts = experts; job.hidden = hidden;
    job.inter = inter; job.std = std; job.int8 = int8; job.payload = payload;
    job.scale = scale; job.zp = zp; job.next = 0;
    pthread_mutex_init(&job.lock, NULL);
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    int started = 0;
    for (int i = 1; i < threads; ++i) {
        if (pthread_create(&tid[started], NULL, layer_worker, &job) == 0) ++started;
    }
    layer_worker(&job);
    for (int i = 0; i < started; ++i) pthread_join(tid[i], NULL);
    pthread_mutex_destroy(&job.lock);
    return 0;
}
