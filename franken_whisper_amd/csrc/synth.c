/*
 * synth.c — deterministic synthetic inputs for tests and benchmarks: seeded
 * random-init weights (N(0, std) drawn in double, rounded to f32 then RNE to
 * f16) and seeded synthetic 16 kHz audio (three sines plus Voss-McCartney pink
 * noise at -20 dBFS RMS, optional digital-silence gaps).
 *
 * Counter-based: element i of tensor `name` depends only on (seed, name, i),
 * through SplitMix64 and Box-Muller, so tensors can be generated in any order
 * and in parallel.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t fnv1a(const char *s) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *s; s++) h = (h ^ (uint8_t)*s) * 0x100000001b3ull;
    return h;
}

static inline double unit_open(uint64_t r) { return ((double)(r >> 11) + 1.0) * 0x1.0p-53; } /* (0,1] */
static inline double unit_half(uint64_t r) { return (double)(r >> 11) * 0x1.0p-53; }        /* [0,1) */

static inline double normal_at(uint64_t key, int64_t i) {
    uint64_t a = splitmix64(key ^ (uint64_t)(2 * i));
    uint64_t b = splitmix64(key ^ (uint64_t)(2 * i + 1) ^ 0xA5A5A5A5A5A5A5A5ull);
    double u1 = unit_open(a), u2 = unit_half(b);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

static inline uint16_t f32_to_f16_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    if (a >= 0x38800000u) {
        uint32_t r = a - (112u << 23);
        r += 0xfffu + ((r >> 13) & 1u);
        r >>= 13;
        return (uint16_t)(sign | (r >= 0x7c00u ? 0x7c00u : r));
    }
    uint32_t e = a >> 23;
    if (e < 102) return sign;
    uint32_t m = (a & 0x7fffffu) | 0x800000u, s = 126u - e;
    uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

static uint64_t tensor_key(uint64_t seed, const char *name) {
    return splitmix64(seed ^ splitmix64(fnv1a(name)));
}

void fws_normal_f32(uint64_t seed, const char *name, double stdv, int64_t n, float *out) {
    uint64_t key = tensor_key(seed, name);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = (float)(stdv * normal_at(key, i));
}

void fws_normal_f16(uint64_t seed, const char *name, double stdv, int64_t n, uint16_t *out) {
    uint64_t key = tensor_key(seed, name);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = f32_to_f16_rne((float)(stdv * normal_at(key, i)));
}

void fws_uniform_i32(uint64_t seed, const char *name, int32_t lo, int32_t hi, int64_t n,
                     int32_t *out) {
    uint64_t key = tensor_key(seed, name);
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo);
    for (int64_t i = 0; i < n; i++) out[i] = lo + (int32_t)(splitmix64(key ^ (uint64_t)i) % span);
}

/* Synthetic 16 kHz mono audio.  Three sines at U(100,4000) Hz with amplitudes
 * U(0.05,0.2) and random phases, plus pink noise (Voss-McCartney, 16 rows)
 * normalised to -20 dBFS RMS.  With gaps != 0 the signal alternates U(3,10) s of
 * sound with U(0.5,2) s of digital silence. */
void fws_audio(uint64_t seed, int64_t n, int gaps, float *out) {
    const double sr = 16000.0;
    uint64_t key = tensor_key(seed, "audio");
    double freq[3], amp[3], ph[3];
    for (int k = 0; k < 3; k++) {
        freq[k] = 100.0 + 3900.0 * unit_half(splitmix64(key ^ (uint64_t)(10 + k)));
        amp[k] = 0.05 + 0.15 * unit_half(splitmix64(key ^ (uint64_t)(20 + k)));
        ph[k] = 6.283185307179586 * unit_half(splitmix64(key ^ (uint64_t)(30 + k)));
    }
    /* pink noise (sequential state) */
    double rows[16];
    double total = 0.0;
    uint64_t st = splitmix64(key ^ 0x51ull);
    for (int r = 0; r < 16; r++) {
        st = splitmix64(st);
        rows[r] = unit_half(st) * 2.0 - 1.0;
        total += rows[r];
    }
    double sumsq = 0.0;
    for (int64_t i = 0; i < n; i++) {
        int64_t c = i + 1;
        int r = 0;
        while (r < 15 && !(c & 1)) { c >>= 1; r++; }
        st = splitmix64(st);
        double nv = unit_half(st) * 2.0 - 1.0;
        total += nv - rows[r];
        rows[r] = nv;
        st = splitmix64(st);
        double white = unit_half(st) * 2.0 - 1.0;
        double p = (total + white) / 17.0;
        out[i] = (float)p;
        sumsq += p * p;
    }
    double rms = sqrt(sumsq / (double)(n > 0 ? n : 1));
    double g = rms > 0 ? 0.1 / rms : 0.0; /* -20 dBFS RMS */
    for (int64_t i = 0; i < n; i++) {
        double t = (double)i / sr, s = 0.0;
        for (int k = 0; k < 3; k++) s += amp[k] * sin(6.283185307179586 * freq[k] * t + ph[k]);
        out[i] = (float)(s + g * out[i]);
    }
    if (gaps) {
        uint64_t gs = splitmix64(key ^ 0x6A9ull);
        int64_t i = 0;
        while (i < n) {
            gs = splitmix64(gs);
            int64_t sound = (int64_t)((3.0 + 7.0 * unit_half(gs)) * sr);
            gs = splitmix64(gs);
            int64_t gap = (int64_t)((0.5 + 1.5 * unit_half(gs)) * sr);
            i += sound;
            for (int64_t j = i; j < i + gap && j < n; j++) out[j] = 0.0f;
            i += gap;
        }
    }
}
