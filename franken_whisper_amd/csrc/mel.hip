// mel.hip — the log-mel frontend (mel::log_mel, mel.rs:1476-1660) on the GPU.
//
// One wave per 400-sample frame, 8 frames per block.  The default two-for-one
// real FFT of the reference (fft_twoforone, mel.rs:648-695) is one complex FFT
// of 200 points: its recursion (cfft, mel.rs:604-646) splits 200 -> 100 -> 50 ->
// 25 by even/odd index, so leaf r (0..7) holds z[r + 8j] with r's bits giving
// the split path, and each leaf is the 5 x 5 radix-5 DFT (radix5_cdft,
// mel.rs:533-577).  The wave evaluates the recursion level by level instead of
// depth first, every output with the reference's expression, so each value is
// bit-identical (f32, no contraction).  Then the power spectrum, the sparse f64
// mel projection (power_and_project, mel.rs:1206-1237), log10_floor_approx
// (mel.rs:1239-1249) and, over the whole output, the max - 8 clamp and
// (x + 4) / 4 normalization (mel.rs:1610-1650).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <mutex>

#include "fw_internal.h"

#define MEL_NFFT 400
#define MEL_HOP 160
#define MEL_NBINS 201
#define MEL_PAD1 480000 // N_SAMPLES_30S
#define MEL_PAD2 200    // N_FFT / 2
#define MEL_FPB 8       // frames (waves) per block
#define MEL_MAXMEL 256  // mel bins a block stages

// Twiddles and window, built on the host with the reference's f64
// transcendentals narrowed to f32 (FftTwiddles::build, DftTable::build,
// hann_window, mel.rs:243-391).
struct MelTables {
    float hann[MEL_NFFT];
    float lcos[4][200], lnsin[4][200]; // split widths 400, 200, 100, 50 (half 200 >> l)
    float c5[25], s5[25], c25[25], s25[25];
};

static void mel_tables_build(MelTables &t) {
    const double PI = 3.14159265358979323846;
    for (int i = 0; i < MEL_NFFT; i++)
        t.hann[i] = (float)(0.5 * (1.0 - cos((2.0 * PI * (double)i) / (double)MEL_NFFT)));
    for (int l = 0; l < 4; l++) {
        const int n = MEL_NFFT >> l, half = n / 2;
        for (int k = 0; k < 200; k++) {
            if (k < half) {
                const double th = (2.0 * PI * (double)k) / (double)n;
                t.lcos[l][k] = (float)cos(th);
                t.lnsin[l][k] = -(float)sin(th);
            } else {
                t.lcos[l][k] = t.lnsin[l][k] = 0.0f;
            }
        }
    }
    for (int k = 0; k < 5; k++)
        for (int j = 0; j < 5; j++) {
            const double th = (2.0 * PI * (double)(k * j)) / 5.0;
            t.c5[k * 5 + j] = (float)cos(th);
            t.s5[k * 5 + j] = (float)sin(th);
            const double th2 = (2.0 * PI * (double)(k * j)) / 25.0;
            t.c25[k * 5 + j] = (float)cos(th2);
            t.s25[k * 5 + j] = (float)sin(th2);
        }
}

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// values.  The FFT stages of a frame touch only that wave's buffers, and a
// wave's LDS operations execute in issue order, so the fences (which keep the
// compiler from moving LDS accesses across) stand in for a block barrier.
__device__ __forceinline__ void mel_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// log10_floor_approx (mel.rs:1239-1249), in f64 then narrowed.
__device__ __forceinline__ float mel_log10_approx(double x) {
    x = x > 1e-10 ? x : 1e-10;
    const uint64_t bits = (uint64_t)__double_as_longlong(x);
    const int64_t ex = (int64_t)((bits >> 52) & 0x7ff) - 1023;
    const double m = __longlong_as_double((long long)((bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull));
    const double t = (m - 1.0) / (m + 1.0);
    const double t2 = t * t;
    const double series = 1.0 + t2 * (1.0 / 3.0 + t2 * (1.0 / 5.0 + t2 * (1.0 / 7.0 + t2 * (1.0 / 9.0))));
    const double ln_m = 2.0 * t * series;
    return (float)(((double)ex * 0.693147180559945309417232121458176568 + ln_m) *
                   (1.0 / 2.302585092994045684017991454684364208));
}

// Nonzero [start, end) bin range of each filter (SparseMelFilters::new), one
// wave per filter: first and last nonzero bin by a wave min / max.
__global__ void __launch_bounds__(256) k_mel_ranges(const float *filters, int n_mel, int2 *ranges) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (m >= n_mel) return;
    const float *row = filters + (size_t)m * MEL_NBINS;
    int a = MEL_NBINS, b = -1;
    for (int k = lane; k < MEL_NBINS; k += 64)
        if (row[k] != 0.0f) {
            a = a < k ? a : k;
            b = k;
        }
    for (int o = 32; o > 0; o >>= 1) {
        const int a2 = __shfl_xor(a, o, 64), b2 = __shfl_xor(b, o, 64);
        a = a < a2 ? a : a2;
        b = b > b2 ? b : b2;
    }
    if (lane == 0) ranges[m] = make_int2(b < 0 ? 0 : a, b < 0 ? 0 : b + 1);
}

// The frames kernel.  Buffers per wave (LDS, floats): A = the windowed frame
// (= the packed complex input z, interleaved), B and C = work arrays.
__global__ void __launch_bounds__(64 * MEL_FPB) k_mel_frames(const float *samples, long long n, long long nf,
                                                             const float *filters, const int2 *ranges, int n_mel,
                                                             const MelTables *__restrict__ gtb, float floor10,
                                                             float *out, float *pmax) {
    // Two buffers per wave, used in turn: frame A -> leaves B -> widths 50 A,
    // 100 B, 200 A -> power B; the mel column then goes to A for the coalesced
    // mel-major store.
    static_assert(MEL_MAXMEL <= 400, "mel column must fit a frame buffer");
    __shared__ float sh[MEL_FPB][2][400];
    __shared__ float wmax[MEL_FPB];
    __shared__ MelTables stb;
    const MelTables *tb = &stb;
    for (int i = threadIdx.x; i < (int)(sizeof(MelTables) / 4); i += blockDim.x)
        ((float *)&stb)[i] = ((const float *)gtb)[i];
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const long long f = (long long)blockIdx.x * MEL_FPB + w;
    float *A = sh[w][0], *B = sh[w][1];
    const long long valid = n + MEL_PAD2;
    const bool live = f < nf;
    const long long off = f * MEL_HOP;
    const bool fft = live && off < valid;
    if (fft) {
        // windowed frame; padded[p] is samples[p - 200] inside the audio, the
        // reflection samples[200 - p] before it (only what exists), else 0
        const long long refl = MEL_PAD2 < (n > 0 ? n - 1 : 0) ? MEL_PAD2 : (n > 0 ? n - 1 : 0);
        const long long avail = valid - off < MEL_NFFT ? valid - off : MEL_NFFT;
        for (int j = lane; j < MEL_NFFT; j += 64) {
            float v = 0.0f;
            if (j < avail) {
                const long long p = off + j;
                float s = 0.0f;
                if (p >= MEL_PAD2) s = p - MEL_PAD2 < n ? samples[p - MEL_PAD2] : 0.0f;
                else if (MEL_PAD2 - p <= refl) s = samples[MEL_PAD2 - p];
                v = tb->hann[j] * s;
            }
            A[j] = v;
        }
    }
    mel_wave_sync();
    if (fft && lane < 40) {
        // leaves: 8 radix-5 DFTs of 25 points, leaf r over z[r + 8 j].  Lane
        // (r, k1) forms both 5-point passes of its column in registers: pass 1
        // and its twiddle for every n2, then pass 2 for every k2 (the outputs
        // k1 + 5 k2 of leaf r, into B at [r][k]).
        const int r = lane / 5, k1 = lane % 5;
        float tr[5], ti[5];
#pragma unroll
        for (int n2 = 0; n2 < 5; n2++) {
            float re = 0.0f, im = 0.0f;
#pragma unroll
            for (int n1 = 0; n1 < 5; n1++) {
                const int zi = r + 8 * (5 * n1 + n2);
                const float xr = A[2 * zi], xi = A[2 * zi + 1];
                const float c = tb->c5[k1 * 5 + n1], s = tb->s5[k1 * 5 + n1];
                re += xr * c + xi * s;
                im += xi * c - xr * s;
            }
            const float c = tb->c25[n2 * 5 + k1], s = tb->s25[n2 * 5 + k1];
            tr[n2] = re * c + im * s;
            ti[n2] = im * c - re * s;
        }
#pragma unroll
        for (int k2 = 0; k2 < 5; k2++) {
            float re = 0.0f, im = 0.0f;
#pragma unroll
            for (int n2 = 0; n2 < 5; n2++) {
                const float c = tb->c5[k2 * 5 + n2], s = tb->s5[k2 * 5 + n2];
                re += tr[n2] * c + ti[n2] * s;
                im += ti[n2] * c - tr[n2] * s;
            }
            const int k = k1 + 5 * k2;
            B[2 * (r * 25 + k)] = re;
            B[2 * (r * 25 + k) + 1] = im;
        }
    }
    // combine levels: width 50 (level 3), 100 (level 2), 200 (level 1).  A node
    // at depth d is the path of its first d splits; its even child takes the
    // next split bit 0.  Leaf r = b1 + 2 b2 + 4 b3 sits at position r in the
    // source buffer; a combined node of width 2h is stored at its own index.
    float *src = B, *dst = A;
    for (int lvl = 3, h = 25, nodes = 4; lvl >= 1; lvl--, h <<= 1, nodes >>= 1) {
        mel_wave_sync();
        if (fft) {
            for (int it = lane; it < nodes * h; it += 64) {
                const int node = it / h, k = it % h;
                // children: even = node, odd = node + nodes (the deeper split bit)
                const float *E = src + 2 * (node * h), *O = src + 2 * ((node + nodes) * h);
                const float re = tb->lcos[lvl][k], im = tb->lnsin[lvl][k];
                const float re_odd = O[2 * k], im_odd = O[2 * k + 1];
                const float e_re = E[2 * k], e_im = E[2 * k + 1];
                float *D = dst + 2 * (node * 2 * h);
                D[2 * k] = e_re + re * re_odd - im * im_odd;
                D[2 * k + 1] = e_im + re * im_odd + im * re_odd;
                D[2 * (k + h)] = e_re - re * re_odd + im * im_odd;
                D[2 * (k + h) + 1] = e_im - re * im_odd - im * re_odd;
            }
        }
        float *tmp = src;
        src = dst;
        dst = tmp;
    }
    mel_wave_sync();
    // src now holds Z (200 complex).  Unpack the two-for-one and take the power
    // of bins 0..200 into dst.
    if (fft) {
        for (int k = lane; k < 200; k += 64) {
            const int km = (200 - k) % 200;
            const float ar = src[2 * k], ai = src[2 * k + 1], br = src[2 * km], bi = src[2 * km + 1];
            const float e_re = 0.5f * (ar + br), e_im = 0.5f * (ai - bi);
            const float o_re = 0.5f * (ai + bi), o_im = 0.5f * (br - ar);
            const float re = tb->lcos[0][k], im = tb->lnsin[0][k];
            const float r0 = e_re + re * o_re - im * o_im;
            const float i0 = e_im + re * o_im + im * o_re;
            dst[k] = r0 * r0 + i0 * i0;
            if (k == 0) {
                const float r1 = e_re - re * o_re + im * o_im;
                const float i1 = e_im - re * o_im - im * o_re;
                dst[200] = r1 * r1 + i1 * i1;
            }
        }
    }
    mel_wave_sync();
    // mel projection, one thread per filter
    float mx = -INFINITY;
    if (live) {
        for (int m = lane; m < n_mel; m += 64) {
            float v = floor10;
            if (fft) {
                const int2 rg = ranges[m];
                const float *row = filters + (size_t)m * MEL_NBINS;
                double sum = 0.0;
                for (int k = rg.x; k < rg.y; k++) sum += (double)dst[k] * (double)row[k];
                v = mel_log10_approx(sum);
            }
            A[m] = v;
            mx = fmaxf(mx, v);
        }
    }
    // block max for the clamp
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) wmax[w] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = wmax[0];
        for (int i = 1; i < MEL_FPB; i++) b = fmaxf(b, wmax[i]);
        pmax[blockIdx.x] = b;
    }
    // mel-major store: runs of the block's consecutive frames per filter
    const long long f0 = (long long)blockIdx.x * MEL_FPB;
    for (int i = threadIdx.x; i < n_mel * MEL_FPB; i += blockDim.x) {
        const int m = i / MEL_FPB, fr = i % MEL_FPB;
        if (f0 + fr < nf) out[(size_t)m * nf + f0 + fr] = sh[fr][0][m];
    }
}

// Global max of the per-block maxima (one block), then the clamp floor.
__global__ void __launch_bounds__(1024) k_mel_floor(const float *pmax, int nb, float *flr) {
    __shared__ float sm[16];
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < nb; i += blockDim.x) mx = fmaxf(mx, pmax[i]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if ((threadIdx.x & 63) == 0) sm[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = sm[0];
        for (int i = 1; i < (int)(blockDim.x >> 6); i++) b = fmaxf(b, sm[i]);
        flr[0] = b - 8.0f;
    }
}

// log_spec = max(log_spec, max - 8); (x + 4) / 4
__global__ void k_mel_norm(float *out, long long total, const float *flr) {
    const float fl = flr[0];
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        float v = out[i];
        v = v < fl ? fl : v;
        out[i] = (v + 4.0f) / 4.0f;
    }
}

#define MEL_TRY(expr)                                                                                   \
    do {                                                                                                \
        hipError_t _e = (expr);                                                                         \
        if (_e != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string(#expr ": ") + hipGetErrorString(_e)); \
    } while (0)

extern "C" int64_t fwhip_mel_frames(int64_t n_samples) {
    if (n_samples < 0) return 0;
    return (n_samples + MEL_PAD1 + 2 * MEL_PAD2 - MEL_NFFT) / MEL_HOP;
}

// The four launches of one log-mel: filter ranges, the frames (log10 power of
// the projection, per-block maxima), the global floor, the normalization.
// `ranges`, `pmax` and `flr` are the scratch (n_mel int2, nb floats, 1 float).
static void mel_launch(hipStream_t st, const float *samples, long long n, long long nf, long long nb,
                       const float *filters, int n_mel, const MelTables *tab, int2 *ranges, float *pmax, float *flr,
                       float *out) {
    const float floor10 = (float)log10(1e-10);
    hipLaunchKernelGGL(k_mel_ranges, dim3((n_mel + 3) / 4), dim3(256), 0, st, filters, n_mel, ranges);
    hipLaunchKernelGGL(k_mel_frames, dim3((unsigned)nb), dim3(64 * MEL_FPB), 0, st, samples, n, nf, filters,
                       (const int2 *)ranges, n_mel, tab, floor10, out, pmax);
    hipLaunchKernelGGL(k_mel_floor, dim3(1), dim3(1024), 0, st, (const float *)pmax, (int)nb, flr);
    const long long total = (long long)n_mel * nf;
    long long g = (total + 255) / 256;
    g = g < 4096 ? g : 4096;
    hipLaunchKernelGGL(k_mel_norm, dim3((unsigned)g), dim3(256), 0, st, out, total, (const float *)flr);
}

// The reference's argument checks (log_mel's InvalidRequest cases) and this
// build's limits, shared by both entry points.
static fwhip_status mel_check(const char *who, fwhip_ctx *c, const float *samples, int64_t n, const float *filters,
                              int32_t n_mel, int32_t n_fft_bins, const float *out) {
    if (!c) return fw_fail(FWHIP_ERR_INVALID, std::string(who) + ": NULL ctx");
    if (n_fft_bins != MEL_NBINS)
        return fw_fail(FWHIP_ERR_INVALID, "mel filterbank has " + std::to_string(n_fft_bins) +
                                              " bins, expected 201 (N_FFT/2+1)");
    if (n_mel <= 0) return fw_fail(FWHIP_ERR_INVALID, "mel filterbank has zero mel bins");
    if (n_mel > MEL_MAXMEL) return fw_fail(FWHIP_ERR_INVALID, std::string(who) + ": more than 256 mel bins");
    if (n < 0 || (n > 0 && !samples) || !filters || !out)
        return fw_fail(FWHIP_ERR_INVALID, std::string(who) + ": NULL buffer or negative length");
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_log_mel(fwhip_ctx *c, const float *samples, int64_t n, const float *filters,
                                      int32_t n_mel, int32_t n_fft_bins, float *out) {
    fwhip_status r = mel_check("fwhip_log_mel", c, samples, n, filters, n_mel, n_fft_bins, out);
    if (r != FWHIP_OK) return r;
    MEL_TRY(hipSetDevice(c->device));
    if (!c->mel_tab) {
        MelTables tb;
        mel_tables_build(tb);
        MEL_TRY(hipMalloc(&c->mel_tab, sizeof(MelTables)));
        MEL_TRY(hipMemcpy(c->mel_tab, &tb, sizeof(MelTables), hipMemcpyHostToDevice));
    }
    const long long nf = fwhip_mel_frames(n);
    const long long nb = (nf + MEL_FPB - 1) / MEL_FPB;
    if (nb > (1ll << 30)) return fw_fail(FWHIP_ERR_INVALID, "fwhip_log_mel: input too long");
    // scratch: filter ranges (int2 each), per-block maxima, the floor
    const size_t need = (size_t)n_mel * 8 + (size_t)nb * 4 + 256;
    if (need > c->mel_scratch_bytes) {
        MEL_TRY(hipStreamSynchronize(c->stream));
        if (c->mel_scratch) MEL_TRY(hipFree(c->mel_scratch));
        c->mel_scratch = nullptr;
        c->mel_scratch_bytes = 0;
        MEL_TRY(hipMalloc(&c->mel_scratch, need));
        c->mel_scratch_bytes = need;
    }
    int2 *ranges = (int2 *)c->mel_scratch;
    float *pmax = (float *)((char *)c->mel_scratch + (size_t)n_mel * 8);
    mel_launch(c->stream, samples, (long long)n, nf, nb, filters, (int)n_mel, (const MelTables *)c->mel_tab, ranges,
               pmax, pmax + nb, out);
    MEL_TRY(hipGetLastError());
    return FWHIP_OK;
}

// ---- allocation-free variant -------------------------------------------------
// For callers that cannot allocate device memory (code under HIP graph capture,
// tight serving loops, harnesses that forbid it): the scratch of the log-mel
// (filter ranges, per-block maxima, the floor) lives in the file-scope device
// array `scratch`, and the window/twiddle tables in `mel_tables_dev`.  Each GPU
// holds its own copy of both until the process ends.  fw_mel_noalloc_setup,
// called by fwhip_init with the device current, resolves their device addresses
// once per device (host code never passes the arrays' names to a kernel: on
// the host they are stand-ins, not device addresses) and uploads the tables.
// Every call on a device shares that device's scratch, which keeps the last
// call's contents; nothing in it needs to start at zero (each launch writes
// every entry it later reads).  Calls that overlap on one GPU race.
#define MEL_SCRATCH_BYTES (512 * 1024)
#define MEL_MAX_DEVICES 64
static __device__ __align__(256) unsigned char scratch[MEL_SCRATCH_BYTES];
static __device__ __align__(256) MelTables mel_tables_dev;

static std::mutex g_noalloc_mu;
static void *g_scratch_ptr[MEL_MAX_DEVICES];
static const MelTables *g_tables_ptr[MEL_MAX_DEVICES];
static int g_noalloc_state[MEL_MAX_DEVICES]; // 0 not set up, 1 ready, -1 set-up failed

// The largest input the scratch holds: frames whose per-block maxima fit next
// to 256 filter ranges and the floor.
static long long mel_noalloc_max_frames() {
    return (long long)((MEL_SCRATCH_BYTES - 256 - MEL_MAXMEL * 8) / 4) * MEL_FPB;
}

void fw_mel_noalloc_setup(int device) {
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (device < 0 || device >= MEL_MAX_DEVICES || g_noalloc_state[device] == 1) return;
    void *p = nullptr, *t = nullptr;
    MelTables tb;
    mel_tables_build(tb);
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p ||
        hipGetSymbolAddress(&t, HIP_SYMBOL(mel_tables_dev)) != hipSuccess || !t ||
        hipMemcpy(t, &tb, sizeof(MelTables), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        g_noalloc_state[device] = -1;
        return;
    }
    g_scratch_ptr[device] = p;
    g_tables_ptr[device] = (const MelTables *)t;
    g_noalloc_state[device] = 1;
}

extern "C" fwhip_status fwhip_log_mel_noalloc(fwhip_ctx *c, const float *samples, int64_t n, const float *filters,
                                              int32_t n_mel, int32_t n_fft_bins, float *out) {
    fwhip_status r = mel_check("fwhip_log_mel_noalloc", c, samples, n, filters, n_mel, n_fft_bins, out);
    if (r != FWHIP_OK) return r;
    const int dev = c->device;
    int state;
    void *sp;
    const MelTables *tp;
    {
        std::lock_guard<std::mutex> lk(g_noalloc_mu);
        state = dev >= 0 && dev < MEL_MAX_DEVICES ? g_noalloc_state[dev] : -1;
        sp = state == 1 ? g_scratch_ptr[dev] : nullptr;
        tp = state == 1 ? g_tables_ptr[dev] : nullptr;
    }
    if (state != 1)
        return fw_fail(FWHIP_ERR_GENERIC, "fwhip_log_mel_noalloc: the device scratch of device " +
                                              std::to_string(dev) + " was not set up by fwhip_init");
    const long long nf = fwhip_mel_frames(n);
    const long long nb = (nf + MEL_FPB - 1) / MEL_FPB;
    const size_t need = (size_t)n_mel * 8 + (size_t)nb * 4 + 256;
    if (nf > mel_noalloc_max_frames() || need > (size_t)MEL_SCRATCH_BYTES)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_log_mel_noalloc: " + std::to_string(nf) +
                                              " frames exceed the allocation-free scratch (at most " +
                                              std::to_string(mel_noalloc_max_frames()) + " frames, " +
                                              std::to_string(MEL_SCRATCH_BYTES) + " bytes); use fwhip_log_mel");
    MEL_TRY(hipSetDevice(dev));
    int2 *ranges = (int2 *)sp;
    float *pmax = (float *)((char *)sp + (size_t)n_mel * 8);
    mel_launch(c->stream, samples, (long long)n, nf, nb, filters, (int)n_mel, tp, ranges, pmax, pmax + nb, out);
    MEL_TRY(hipGetLastError());
    return FWHIP_OK;
}
