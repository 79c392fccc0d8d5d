// fw_dec.h — device helpers shared by the decoder kernels: the decoder
// LayerNorm (+ int8 activation quantizer) of one row per wave, and the
// argmax keys and suppress mask of process_logits.
#pragma once
#include "fw_kernels.h"

// A 16-byte global load marked non-temporal.  Every decode step reads all of
// its weights and cross K/V again; on the f16 arm that is 647 MB a step
// (10 streams), past the 256 MB last-level cache, so a cyclic sweep would keep
// none of it.  Loading the cross K/V rows and the logits head's weights
// (440 MB) this way leaves the cache to the layer weights, which then stay
// from one step to the next: 10-stream step 403 -> 384 us.
__device__ __forceinline__ uint4 fw_ld_stream(const void *p) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v q = __builtin_nontemporal_load((const u4v *)p);
    return make_uint4(q.x, q.y, q.z, q.w);
}

// ---------------------------------------------------------------------------
// LayerNorm (nn.rs:4455-4545: f64 mean/var, ((x-mean)*inv)*w + b rounded to
// f32) of one stream row per wave, then the decoder activation quantizer of
// the normalized row (per-row amax/127, add-trunc body, exact n%8 tail) into
// the int8 activation buffer.  y may be NULL (int8-only consumers), xq may be
// NULL (f32-only consumers).  4 rows per block; lane l holds the float4
// groups l, l+64, ... (NV of them, d <= 256*NV, d % 4 == 0).  Every load of
// x, w and b is issued before the first use, so the row costs one memory
// round trip; the reductions run on DPP lane moves.
// Row r whose values xv (lane l: float4 groups l, l+64, ...; ok = in range)
// are already loaded or in flight.
// LayerNorm weight and bias groups of lane l (as the row values).
template <int NV>
__device__ __forceinline__ void fw_ln_load_wb(const bool (&ok)[NV], const float *w, const float *b, float4 (&wv)[NV],
                                              float4 (&bv)[NV], int lane) {
    const float4 *w4 = (const float4 *)w, *b4 = (const float4 *)b;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int c = ok[k] ? lane + k * 64 : 0;
        wv[k] = w4[c];
        bv[k] = b4[c];
    }
}

// The reference's sequential f64 loops over a row held as above (element
// 4 (l + 64 k) + j in lane l, component j of xv[k]; d = 4 n4):
// SQ = false: sum of (f64)x; SQ = true: sum of ((f64)x - mean)^2
// (nn.rs:4425-4438).  Every lane forms its terms into the wave's LDS slot
// (one slot for each of the block's first 4 waves: only waves 0-3 may call
// it), then lane 0 adds them in index order, each batch of the slot's reads
// issued while the previous batch is added (the chain of dependent f64 adds
// is the floor; an LDS read costs the wave the same for one lane as for 64,
// so the reads go 16 bytes at a time, a batch ahead), and the sum is
// broadcast.  Uniform; every lane of the wave must call it.
#define FW_SEQ_NB 8
__device__ __forceinline__ void fw_seq_ld(const double2 *t2, int i, double2 (&a)[FW_SEQ_NB]) {
#pragma unroll
    for (int u = 0; u < FW_SEQ_NB; u++) a[u] = t2[i + u];
}
__device__ __forceinline__ double fw_seq_add(double s, const double2 (&a)[FW_SEQ_NB]) {
#pragma unroll
    for (int u = 0; u < FW_SEQ_NB; u++) {
        s = s + a[u].x;
        s = s + a[u].y;
    }
    return s;
}
// the wave's slot (one array per row width, shared by both sums)
template <int NV>
__device__ __forceinline__ double2 *fw_seq_slot() {
    __shared__ double2 fw_seq_tm[4][128 * NV];
    return fw_seq_tm[(threadIdx.x >> 6) & 3];
}
template <int NV, bool SQ>
__device__ __forceinline__ double fw_row_seq_sum(const float4 (&xv)[NV], int n4, double mean) {
    const int lane = threadIdx.x & 63;
    double2 *tm = fw_seq_slot<NV>();
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if (lane + 64 * k < n4) {
            const double v[4] = {(double)xv[k].x, (double)xv[k].y, (double)xv[k].z, (double)xv[k].w};
            double t[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (SQ) {
                    const double u = v[j] - mean;
                    t[j] = u * u;
                } else {
                    t[j] = v[j];
                }
            }
            tm[2 * (lane + 64 * k)] = make_double2(t[0], t[1]);
            tm[2 * (lane + 64 * k) + 1] = make_double2(t[2], t[3]);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    double s = 0.0;
    if (lane == 0) {
        const int n2 = 2 * n4, nb = n2 / FW_SEQ_NB; // double2 terms, whole batches
        double2 a[FW_SEQ_NB], b[FW_SEQ_NB];
        int i = 0;
        if (nb > 0) fw_seq_ld(tm, 0, a);
        for (; i + 2 <= nb; i += 2) {
            fw_seq_ld(tm, (i + 1) * FW_SEQ_NB, b);
            s = fw_seq_add(s, a);
            if (i + 2 < nb) fw_seq_ld(tm, (i + 2) * FW_SEQ_NB, a);
            s = fw_seq_add(s, b);
        }
        if (i < nb) s = fw_seq_add(s, a);
        for (int j = nb * FW_SEQ_NB; j < n2; j++) {
            s = s + tm[j].x;
            s = s + tm[j].y;
        }
    }
    s = __shfl(s, 0, 64);
    // (the slot is rewritten by the wave's next call; its reads above come first)
    __builtin_amdgcn_wave_barrier();
    return s;
}

// Whether every partial sum of the row's (f64)x, in any order, is exact:
// each value is a multiple of g = 2^(emin - 150) (emin the smallest biased
// exponent of a nonzero value, 1 for subnormals) and every partial sum is
// below d * 2^(emax - 126) in magnitude, so all of them are integers times g
// below 2^53 g when emax - emin <= 29 - ceil(log2 d).  Then the wave's tree
// sum equals the sequential one bit for bit.  Non-finite values say no.
template <int NV>
__device__ __forceinline__ bool fw_row_sum_exact(const float4 (&xv)[NV], const bool (&ok)[NV], int d) {
    float emx = 0.0f, nmn = -255.0f; // max exponent, -(min exponent)
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if (ok[k]) {
            const uint32_t u[4] = {__float_as_uint(xv[k].x), __float_as_uint(xv[k].y), __float_as_uint(xv[k].z),
                                   __float_as_uint(xv[k].w)};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t a = u[j] & 0x7fffffffu;
                if (a) {
                    const uint32_t e = (a >> 23) > 1u ? (a >> 23) : 1u;
                    emx = fmaxf(emx, (float)e);
                    nmn = fmaxf(nmn, -(float)e);
                }
            }
        }
    }
    emx = fw_dpp_wave_max(emx);
    nmn = fw_dpp_wave_max(nmn);
    if (emx == 0.0f) return true; // every value is zero
    const int lg = 32 - __builtin_clz((unsigned)(d > 1 ? d - 1 : 1)); // ceil(log2 d)
    return emx < 255.0f && (int)emx + (int)nmn <= 29 - lg;
}

// The same with the weight and bias groups already loaded (or in flight).
// SEQ: the mean and variance sums are the reference's sequential f64 loops
// (bit for bit, whatever the row); else the mean is the wave's tree sum (the
// same bits whenever fw_row_sum_exact holds) and the variance the tree sum
// of per-lane partials, which can differ from the sequential sum in its last
// bits.
template <int NV, bool SEQ = false>
__device__ __forceinline__ void fw_ln_quant_core(float4 (&xv)[NV], const bool (&ok)[NV], const float4 (&wv)[NV],
                                                 const float4 (&bv)[NV], float *y, int d, int r, int8_t *xq,
                                                 float *xs, int lane) {
    double mean;
    if (SEQ && !fw_row_sum_exact<NV>(xv, ok, d)) {
        mean = fw_row_seq_sum<NV, false>(xv, d >> 2, 0.0) / (double)d;
    } else {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < NV; k++)
            if (ok[k]) s += ((double)xv[k].x + (double)xv[k].y) + ((double)xv[k].z + (double)xv[k].w);
        mean = fw_dpp_wave_sum_f64(s) / (double)d;
    }
    double var;
    if constexpr (SEQ) {
        var = fw_row_seq_sum<NV, true>(xv, d >> 2, mean) / (double)d;
    } else {
        double v = 0.0;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            if (ok[k]) {
                const double a = (double)xv[k].x - mean, bb = (double)xv[k].y - mean;
                const double c = (double)xv[k].z - mean, e = (double)xv[k].w - mean;
                v += (a * a + bb * bb) + (c * c + e * e);
            }
        }
        var = fw_dpp_wave_sum_f64(v) / (double)d;
    }
    const double inv = 1.0 / sqrt(var + (double)1e-5f);
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        float4 o;
        o.x = (float)((((double)xv[k].x - mean) * inv) * (double)wv[k].x + (double)bv[k].x);
        o.y = (float)((((double)xv[k].y - mean) * inv) * (double)wv[k].y + (double)bv[k].y);
        o.z = (float)((((double)xv[k].z - mean) * inv) * (double)wv[k].z + (double)bv[k].z);
        o.w = (float)((((double)xv[k].w - mean) * inv) * (double)wv[k].w + (double)bv[k].w);
        xv[k] = o;
        if (ok[k]) {
            m = fmaxf(m, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
            if (y) ((float4 *)(y + (size_t)r * d))[lane + k * 64] = o;
        }
    }
    if (!xq) return;
    m = fw_dpp_wave_max(m);
    const float sc = fmaxf(m, 1e-9f) / 127.0f;
    const float iv = 1.0f / sc;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if (ok[k]) {
            const int i = (lane + k * 64) * 4;
            const uint32_t q = (uint32_t)(uint8_t)fw_q8_avx(xv[k].x, iv, i, d) |
                               ((uint32_t)(uint8_t)fw_q8_avx(xv[k].y, iv, i + 1, d) << 8) |
                               ((uint32_t)(uint8_t)fw_q8_avx(xv[k].z, iv, i + 2, d) << 16) |
                               ((uint32_t)(uint8_t)fw_q8_avx(xv[k].w, iv, i + 3, d) << 24);
            *(uint32_t *)(xq + (size_t)r * d + i) = q;
        }
    }
    if (lane == 0) xs[r] = sc;
}

template <int NV, bool SEQ = false>
__device__ __forceinline__ void fw_ln_quant_vals(float4 (&xv)[NV], const bool (&ok)[NV], float *y, const float *w,
                                                 const float *b, int d, int r, int8_t *xq, float *xs, int lane) {
    float4 wv[NV], bv[NV];
    fw_ln_load_wb<NV>(ok, w, b, wv, bv, lane);
    fw_ln_quant_core<NV, SEQ>(xv, ok, wv, bv, y, d, r, xq, xs, lane);
}


// ---------------------------------------------------------------------------
// Order-preserving argmax key: larger value first, then smaller index; 0 means
// "no candidate" (masked, -inf or NaN never compare greater, as in the
// reference's strict '>' scan).  -0.0 and +0.0 compare equal under '>', so the
// first of them wins (argmax_idx, decode.rs:1708-1770): both map to one key.
__device__ __forceinline__ unsigned long long am_key(float v, int idx) {
    if (!(v > -INFINITY)) return 0ull;
    uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_max_u64(unsigned long long k) {
    const uint32_t lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)k, CTRL, 0xf, 0xf, false);
    const uint32_t hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(k >> 32), CTRL, 0xf, 0xf, false);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    return o > k ? o : k;
}
// max over each 16-lane row (every lane of the row gets it), DPP moves only
__device__ __forceinline__ unsigned long long row16_max_u64(unsigned long long k) {
    k = dpp_max_u64<FW_DPP_XOR1>(k);
    k = dpp_max_u64<FW_DPP_XOR2>(k);
    k = dpp_max_u64<FW_DPP_HALF_MIRROR>(k);
    return dpp_max_u64<FW_DPP_MIRROR>(k);
}
// max over the wave (every lane gets it)
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
    k = row16_max_u64(k);
    const unsigned long long r0 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 0) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 0);
    const unsigned long long r1 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 16) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 16);
    const unsigned long long r2 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 32) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 32);
    const unsigned long long r3 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 48) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 48);
    const unsigned long long a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
    return a > b ? a : b;
}

// The suppress set of process_logits in no-timestamps mode (decode.rs:702-867).
__device__ __forceinline__ bool dec_masked(int i, const fwhip_filter &f, int initial) {
    if (initial && (i == f.eot || i == f.space_token)) return true;
    if (i >= f.timestamp_begin) return true;
    if (i == f.no_timestamps || i == f.sot || i == f.no_speech || i == f.solm || i == f.translate ||
        i == f.transcribe || i == f.sot_prev)
        return true;
    if (i >= f.sot + 1 && i <= f.sot + f.n_languages) return true;
    return false;
}

// ---------------------------------------------------------------------------
// The same sequential f32 sum ((0 + v[0]) + v[1]) + ... of n <= 64 * SW_MAXC
// values v[i] >= 0 (finite, in LDS, readable up to index (n+3) & ~3), by one
// whole wave, bit-identical to the one-thread loop.
//
// While a running sum s stays in one binade [2^k, 2^(k+1)] its bit pattern
// moves by integers: s + e rounds to the grid of ulp 2^(k-23), and the step
// depends on s only through the parity of its last bit (ties go to even).  So
// a lane's chunk of c consecutive values acts, on any start in binade k, as
// bits -> bits + D[bits & 1], and running the chunk's own f32 adds from the
// two lowest starts 2^k and 2^k + ulp gives D[0] and D[1] exactly.
//  1. lane l takes values [l*c, l*c + c) (c = n/64 rounded up to 4), sums
//     them roughly and a wave scan gives its rough start P;
//  2. a lane whose rough range [P, P + chunk] sits inside one binade with a
//     2^-10 margin runs its chunk from both starts (else it is left to step 4);
//  3. consecutive such lanes of one binade compose their (D[0], D[1]) maps in
//     a segmented wave scan: run [a, b] maps parity p to D[p] of the whole run;
//  4. walking the runs in order, a run applies when the exact s lies in its
//     binade and s + D stays <= 2^(k+1) (monotone sums: then every partial
//     sum of the run stayed in the binade); otherwise its values are added one
//     by one, as the reference does.
// Correctness rests on step 4's exact check alone; steps 1-2 only choose
// which lanes to try.  Every lane of the wave must call it (n uniform).
#define SW_MAXC 24
__device__ __forceinline__ float fw_seq_sum_wave(const float *v, int n) {
    const int lane = threadIdx.x & 63;
    const int c = ((((n + 63) >> 6) + 3) & ~3) > 0 ? ((((n + 63) >> 6) + 3) & ~3) : 4; // values per lane, <= SW_MAXC
    const int n4 = (n + 3) >> 2;                                                     // readable float4 groups
    float e[SW_MAXC];
#pragma unroll
    for (int q = 0; q < SW_MAXC / 4; q++) {
        const int g = (lane * c >> 2) + q; // float4 group of this lane's chunk
        float4 x = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (4 * q < c && g < n4) x = ((const float4 *)v)[g];
        const int i0 = lane * c + 4 * q;
        e[4 * q + 0] = 4 * q + 0 < c && i0 + 0 < n ? x.x : 0.0f;
        e[4 * q + 1] = 4 * q + 1 < c && i0 + 1 < n ? x.y : 0.0f;
        e[4 * q + 2] = 4 * q + 2 < c && i0 + 2 < n ? x.z : 0.0f;
        e[4 * q + 3] = 4 * q + 3 < c && i0 + 3 < n ? x.w : 0.0f;
    }
    // 1. rough chunk sum and rough start
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < SW_MAXC; i++) t += e[i];
    float inc = t;
#pragma unroll
    for (int dlt = 1; dlt < 64; dlt <<= 1) {
        const float y = __shfl_up(inc, dlt, 64);
        if (lane >= dlt) inc += y;
    }
    const float P = inc - t;
    // 2. the chunk's map on its guessed binade
    const uint32_t pb = __float_as_uint(P);
    const int ex = (int)(pb >> 23);
    const uint32_t lo = (uint32_t)ex << 23, hi = (uint32_t)(ex + 1) << 23;
    bool ok = ex >= 1 && ex <= 253 && P >= __uint_as_float(lo) * 1.0009765625f &&
              P + t <= __uint_as_float(hi) * 0.9990234375f;
    float s0 = __uint_as_float(lo), s1 = __uint_as_float(lo + 1);
#pragma unroll
    for (int i = 0; i < SW_MAXC; i++) {
        s0 = s0 + e[i];
        s1 = s1 + e[i];
    }
    ok = ok && __float_as_uint(s0) <= hi && __float_as_uint(s1) <= hi;
    int d0 = (int)(__float_as_uint(s0) - lo), d1 = (int)(__float_as_uint(s1) - (lo + 1));
    // 3. runs: consecutive ok lanes of one binade; any other lane is a run of its own
    const uint32_t key = ok ? lo : (0x80000000u | (uint32_t)lane);
    const uint32_t kprev = __shfl_up(key, 1, 64);
    const bool head = lane == 0 || key != kprev;
    int rs = head ? lane : 0; // first lane of this lane's run
#pragma unroll
    for (int dlt = 1; dlt < 64; dlt <<= 1) {
        const int y = __shfl_up(rs, dlt, 64);
        if (lane >= dlt) rs = max(rs, y);
    }
#pragma unroll
    for (int dlt = 1; dlt < 64; dlt <<= 1) {
        const int a0 = __shfl_up(d0, dlt, 64), a1 = __shfl_up(d1, dlt, 64);
        if (lane - dlt >= rs) {
            // [.., lane - dlt] then [.., lane]
            const int n0 = a0 + ((a0 & 1) ? d1 : d0);
            const int n1 = a1 + (((1 + a1) & 1) ? d1 : d0);
            d0 = n0;
            d1 = n1;
        }
    }
    // 4. walk the runs (uniform)
    unsigned long long heads = __builtin_amdgcn_ballot_w64(head);
    float s = 0.0f;
    while (heads) {
        const int a = __builtin_ctzll(heads);
        heads &= heads - 1;
        const int b = heads ? __builtin_ctzll(heads) - 1 : 63;
        const bool rok = __builtin_amdgcn_readlane((int)ok, b) != 0;
        bool done = false;
        if (rok) {
            const uint32_t rlo = (uint32_t)__builtin_amdgcn_readlane((int)lo, b), rhi = rlo + (1u << 23);
            const uint32_t sb = __float_as_uint(s);
            const uint32_t D = (uint32_t)((sb & 1) ? __builtin_amdgcn_readlane(d1, b) : __builtin_amdgcn_readlane(d0, b));
            if (sb >= rlo && sb < rhi && sb + D <= rhi) {
                s = __uint_as_float(sb + D);
                done = true;
            }
        }
        if (!done) {
            // the run's values one by one, in order: each lane's chunk is read
            // again from LDS (one broadcast address per read, all reads issued
            // before the adds); values past the chunk or past n count as +0,
            // which leaves the non-negative s unchanged
            for (int q = a; q <= b; q++) {
                float4 r[SW_MAXC / 4];
                if (c == SW_MAXC && (q + 1) * c <= n) {
                    // a whole chunk of SW_MAXC values (the usual case)
#pragma unroll
                    for (int i = 0; i < SW_MAXC / 4; i++) r[i] = ((const float4 *)v)[(q * c >> 2) + i];
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int i = 0; i < SW_MAXC / 4; i++) {
                        s = s + r[i].x;
                        s = s + r[i].y;
                        s = s + r[i].z;
                        s = s + r[i].w;
                    }
                    continue;
                }
#pragma unroll
                for (int i = 0; i < SW_MAXC / 4; i++) {
                    const int g = (q * c >> 2) + i;
                    r[i] = 4 * i < c && g < n4 ? ((const float4 *)v)[g] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                float x[SW_MAXC];
#pragma unroll
                for (int i = 0; i < SW_MAXC / 4; i++) {
                    const int i0 = q * c + 4 * i;
                    x[4 * i + 0] = i0 + 0 < n ? r[i].x : 0.0f;
                    x[4 * i + 1] = i0 + 1 < n ? r[i].y : 0.0f;
                    x[4 * i + 2] = i0 + 2 < n ? r[i].z : 0.0f;
                    x[4 * i + 3] = i0 + 3 < n ? r[i].w : 0.0f;
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < SW_MAXC; i++) s = s + x[i];
            }
        }
    }
    return s;
}
