// dec_gemv16.hip — the f16 decoder arm's GEMVs for a cohort of streams (gfx950).
//
// gemv_f16 (nn.rs:2346-2460) computes y[o] = dot_f16c(W[o, :], x) + b[o] with
// dot_f16c's fixed association (nn.rs:1983-2051): 32 partial sums ("slots")
// j = 8k + l (accumulator k = 0..3, lane l = 0..7), slot j an FMA chain over
// element 32c + j of every 32-wide chunk c in ascending c; then per l
// t_l = (a0 + a1) + (a2 + a3) and ((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)).
// Rows need K % 64 == 0 here (every large-v3-turbo and tiny.en projection), so
// there is no 8-chunk or scalar tail.
//
// The weights are shared by the cohort, so one weight element feeds one FMA
// per stream, and the cost is the FMAs plus the operand traffic that feeds
// them.  Layout of the work:
//  - LPR lanes per row ("row group"); lane p = kh * 8 + l owns the CPL = 32 / LPR
//    slots 8 (kh * CPL + kk) + l, kk = 0..CPL-1, so the first step of the slot
//    tree (a0 + a1, and (a0 + a1) + (a2 + a3) at CPL = 4) is in registers and
//    the rest is log2(LPR) lane exchanges;
//  - each lane carries R rows of its row group for the same slots, so one
//    activation value read from LDS feeds R FMAs (LDS return bandwidth, not
//    the FMA rate, limited the one-row-per-lane form: 4 bytes per FMA);
//  - the streams of a block (SB of them, grid.y splits larger cohorts) are
//    staged once in LDS as [chunk][stream][32], each chunk's 32 values permuted
//    so lane p reads its CPL slots as one contiguous LDS load; with LayerNorm
//    weights the staged rows are LN(x) (the decoder LayerNorm, one wave per
//    row, fused so the normalized rows never go through HBM);
//  - weights are repacked once ("slot order", fw_launch_pack_gemv16) so a
//    lane's 16-byte load is 8 / CPL consecutive chunks of its slots and a row
//    group's load is LPR * 16 contiguous bytes;
//  - blocks walk tiles of rows, loading the next batch of weight groups while
//    the current one is multiplied (the batches of consecutive tiles form one
//    pipeline), so a block streams weights at a steady rate;
//  - the epilogue (bias, residual add or GELU) spreads the cohort's outputs of
//    a row over the row group's lanes; residual rows are read at tile start.
//  - with keys, the block also forms per-tile argmax keys of the filtered
//    logits (process_logits' no-timestamps suppress set, first-index strict
//    '>' argmax; decode.rs:702-867, 1708-1780), so the logits need no second
//    pass before the argmax.
#include <type_traits>

#include "fw_dec.h"

namespace {

#ifndef G16_BG_N
#define G16_BG_N 4
#endif
constexpr int G16_BG = G16_BG_N; // weight groups per pipelined batch

template <int LPR>
struct G16 {
    static constexpr int CPL = 32 / LPR; // slots per lane
    static constexpr int CPG = 8 / CPL;  // chunks per 16-byte weight group
    static constexpr int RG = 64 / LPR;  // row groups per wave
};

// LDS position of element e (0..31) of a chunk: lane p's CPL slots contiguous.
template <int LPR>
__device__ __forceinline__ int g16_pos(int e) {
    constexpr int CPL = G16<LPR>::CPL;
    const int k = e >> 3, l = e & 7;
    return ((k / CPL) * 8 + l) * CPL + (k % CPL);
}

template <int LPR, int R, int SB, int WPB, bool LN, bool KEYS>
__global__ void __launch_bounds__(64 * WPB) k_gemv16(const uint16_t *__restrict__ Wp, const float *__restrict__ bias,
                                                    const float *__restrict__ x, float *y, int N, int K, int ns,
                                                    int ldy, int mode, const float *__restrict__ gelu_tab,
                                                    const float *__restrict__ lnw, const float *__restrict__ lnb,
                                                    fwhip_filter filt, int use_filter, const int *initialp,
                                                    unsigned long long *keys) {
    constexpr int CPL = G16<LPR>::CPL, CPG = G16<LPR>::CPG, RG = G16<LPR>::RG;
    constexpr int RPW = RG * R, RPT = RPW * WPB, BG = G16_BG;
    extern __shared__ __align__(16) float xs[]; // [nc][SB][32]
    __shared__ unsigned long long wkey[WPB][SB];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int p = lane % LPR, rg = lane / LPR;
    const int nc = K >> 5, G = nc / CPG;
    const int s0 = blockIdx.y * SB, sn = ns - s0 < SB ? ns - s0 : SB;
    const int ntile = (N + RPT - 1) / RPT;

    // ---- the first tile's weights are requested before the rows are staged
    const int initial = KEYS && use_filter ? *initialp : 0;
    const int nb = (G + BG - 1) / BG; // batches per tile
    int tile = blockIdx.x;
    auto wptr = [&](int t, int r) -> const uint4 * {
        const int row = t * RPT + wave * RPW + r * RG + rg;
        return (const uint4 *)(Wp + (size_t)(row < N ? row : N - 1) * K) + p;
    };
    uint4 nxt[BG][R];
    auto load_batch = [&](int t, int b) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            const uint4 *w = wptr(t, r);
#pragma unroll
            for (int i = 0; i < BG; i++) {
                const int g = b * BG + i;
                // (unconditional: a partial last batch re-reads group G - 1, unused,
                // so no load sits behind a branch and the waits count exactly)
                // (the logits head's weights are read once per step: streamed)
                if constexpr (KEYS) nxt[i][r] = fw_ld_stream(w + (size_t)(g < G ? g : G - 1) * LPR);
                else nxt[i][r] = w[(size_t)(g < G ? g : G - 1) * LPR];
            }
        }
    };
    if (tile < ntile) load_batch(tile, 0);

    // ---- stage the block's stream rows (or their LayerNorm) into LDS
    if constexpr (LN) {
        // K <= 1280: five float4 groups per lane cover a row
        for (int sl = wave; sl < SB; sl += WPB) {
            float4 xv[5];
            bool ok[5];
            const int n4 = K >> 2;
#pragma unroll
            for (int q = 0; q < 5; q++) {
                const int i = lane + q * 64;
                ok[q] = i < n4;
                xv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (sl < sn) xv[q] = ((const float4 *)(x + (size_t)(s0 + sl) * K))[ok[q] ? i : 0];
            }
            if (sl < sn) fw_ln_quant_vals<5>(xv, ok, nullptr, lnw, lnb, K, 0, nullptr, nullptr, lane);
#pragma unroll
            for (int q = 0; q < 5; q++) {
                if (ok[q]) {
                    const int e0 = (lane + q * 64) * 4, c = e0 >> 5;
                    float *dst = xs + ((size_t)c * SB + sl) * 32;
                    const float v[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
#pragma unroll
                    for (int t = 0; t < 4; t++) dst[g16_pos<LPR>((e0 + t) & 31)] = sl < sn ? v[t] : 0.0f;
                }
            }
        }
    } else {
        const int n4 = K >> 2, tot = SB * n4;
        for (int i = threadIdx.x; i < tot; i += 64 * WPB) {
            const int sl = i / n4, c4 = i - sl * n4;
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (sl < sn) v = ((const float4 *)(x + (size_t)(s0 + sl) * K))[c4];
            const int e0 = c4 * 4, c = e0 >> 5;
            float *dst = xs + ((size_t)c * SB + sl) * 32;
            dst[g16_pos<LPR>((e0 + 0) & 31)] = v.x;
            dst[g16_pos<LPR>((e0 + 1) & 31)] = v.y;
            dst[g16_pos<LPR>((e0 + 2) & 31)] = v.z;
            dst[g16_pos<LPR>((e0 + 3) & 31)] = v.w;
        }
    }

    __syncthreads();
    for (; tile < ntile; tile += gridDim.x) {
        const int rowb = tile * RPT + wave * RPW + rg;
        // residual rows for this tile, read before the multiply
        float yo[R][SB];
        if (mode == 1) {
#pragma unroll
            for (int r = 0; r < R; r++)
#pragma unroll
                for (int sl = 0; sl < SB; sl++) {
                    const int row = rowb + r * RG;
                    yo[r][sl] = (row < N && sl < sn && sl % LPR == p) ? y[(size_t)(s0 + sl) * ldy + row] : 0.0f;
                }
        }
        float acc[R][SB][CPL];
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
            for (int sl = 0; sl < SB; sl++)
#pragma unroll
                for (int kk = 0; kk < CPL; kk++) acc[r][sl][kk] = 0.0f;
        // LDS reads run one chunk ahead of the FMAs (xv[0] / xv[1] alternate),
        // so a chunk's multiplies never wait on its own activation loads
        float xv[2][SB][CPL];
        auto load_x = [&](int c, float (&dst)[SB][CPL]) {
            const float *xc = xs + (size_t)c * SB * 32 + p * CPL;
#pragma unroll
            for (int sl = 0; sl < SB; sl++) {
                if constexpr (CPL == 4) {
                    const float4 t = *(const float4 *)(xc + sl * 32);
                    dst[sl][0] = t.x; dst[sl][1] = t.y; dst[sl][2] = t.z; dst[sl][3] = t.w;
                } else if constexpr (CPL == 2) {
                    const float2 t = *(const float2 *)(xc + sl * 32);
                    dst[sl][0] = t.x; dst[sl][1] = t.y;
                } else {
                    dst[sl][0] = xc[sl * 32];
                }
            }
        };
        // multiply the groups of one batch (weights wb in registers); a full
        // batch has no guards (fixed registers, straight-line FMAs), the tail
        // batch skips groups past G
        auto mul = [&](const uint4 (&wb)[BG][R], int b, int nbg, auto tail_tag) {
            constexpr bool TAIL = decltype(tail_tag)::value;
            load_x(b * BG * CPG, xv[0]);
#pragma unroll
            for (int i = 0; i < BG; i++) {
                if (TAIL && i >= nbg) break;
#pragma unroll
                for (int cc = 0; cc < CPG; cc++) {
                    const int c = (b * BG + i) * CPG + cc;
                    const int cur_x = (i * CPG + cc) & 1;
                    if (cc + 1 < CPG || (TAIL ? i + 1 < nbg : i + 1 < BG)) load_x(c + 1, xv[cur_x ^ 1]);
                    float wf[R][CPL];
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        const uint32_t u[4] = {wb[i][r].x, wb[i][r].y, wb[i][r].z, wb[i][r].w};
#pragma unroll
                        for (int kk = 0; kk < CPL; kk++) {
                            const int f = cc * CPL + kk;
                            wf[r][kk] = fw_h2f((uint16_t)(u[f >> 1] >> ((f & 1) * 16)));
                        }
                    }
#pragma unroll
                    for (int sl = 0; sl < SB; sl++)
#pragma unroll
                        for (int r = 0; r < R; r++)
#pragma unroll
                            for (int kk = 0; kk < CPL; kk++)
                                acc[r][sl][kk] = __builtin_fmaf(wf[r][kk], xv[cur_x][sl][kk], acc[r][sl][kk]);
                }
            }
        };
        // one pipelined batch: its weights move out of the in-flight buffer
        // and the next batch (this tile's, or the block's next tile's first) is
        // requested before the multiply
        auto batch = [&](int b, int nbg, auto tail_tag) {
            uint4 cur[BG][R];
#pragma unroll
            for (int i = 0; i < BG; i++)
#pragma unroll
                for (int r = 0; r < R; r++) cur[i][r] = nxt[i][r];
            if (b + 1 < nb) load_batch(tile, b + 1);
            else if (tile + (int)gridDim.x < ntile) load_batch(tile + gridDim.x, 0);
            mul(cur, b, nbg, tail_tag);
        };
        const int nfull = G / BG;
        for (int b = 0; b < nfull; b++) batch(b, BG, std::false_type{});
        if (nfull < nb) batch(nfull, G - nfull * BG, std::true_type{});
        // ---- slot tree, then the epilogue
        unsigned long long kmax[SB];
#pragma unroll
        for (int sl = 0; sl < SB; sl++) kmax[sl] = 0ull;
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = rowb + r * RG;
            const bool ok = row < N;
            const float bv = (bias && ok) ? bias[row] : 0.0f;
            const bool masked = KEYS && (!ok || (use_filter && dec_masked(row, filt, initial)));
#pragma unroll
            for (int sl = 0; sl < SB; sl++) {
                float v;
                if constexpr (CPL == 4) v = (acc[r][sl][0] + acc[r][sl][1]) + (acc[r][sl][2] + acc[r][sl][3]);
                else if constexpr (CPL == 2) v = acc[r][sl][0] + acc[r][sl][1];
                else v = acc[r][sl][0];
                if constexpr (LPR == 32) {
                    v = v + __shfl_xor(v, 8, 64);
                    v = v + __shfl_xor(v, 16, 64);
                } else if constexpr (LPR == 16) {
                    v = v + __shfl_xor(v, 8, 64);
                }
                v = v + __shfl_xor(v, 1, 64);
                v = v + __shfl_xor(v, 2, 64);
                v = v + __shfl_xor(v, 4, 64);
                if (bias) v = v + bv;
                if constexpr (KEYS) {
                    if (!masked && sl < sn) {
                        const unsigned long long kv = am_key(v, row);
                        kmax[sl] = kv > kmax[sl] ? kv : kmax[sl];
                    }
                }
                if (ok && sl < sn && sl % LPR == p) {
                    float *yp = y + (size_t)(s0 + sl) * ldy + row;
                    if (mode == 1) *yp = yo[r][sl] + v;
                    else if (mode == 2) *yp = fw_gelu(v, gelu_tab);
                    else *yp = v;
                }
            }
        }
        if constexpr (KEYS) {
#pragma unroll
            for (int sl = 0; sl < SB; sl++) {
                const unsigned long long k = wave_max_u64(kmax[sl]);
                if (lane == 0) wkey[wave][sl] = k;
            }
            __syncthreads();
            if (threadIdx.x < SB && (int)threadIdx.x < sn) {
                unsigned long long m = wkey[0][threadIdx.x];
#pragma unroll
                for (int w = 1; w < WPB; w++) m = wkey[w][threadIdx.x] > m ? wkey[w][threadIdx.x] : m;
                keys[(size_t)(s0 + threadIdx.x) * ntile + tile] = m;
            }
            __syncthreads();
        }
    }
}

__global__ void __launch_bounds__(256) k_pack_gemv16(const uint16_t *W, uint16_t *Wp, int N, int K, int LPR) {
    const int CPL = 32 / LPR, CPG = 8 / CPL;
    const size_t total = (size_t)N * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t r = i / K;
        const int k = (int)(i - r * K);
        const int c = k >> 5, e = k & 31, ks = e >> 3, l = e & 7;
        const int pl = (ks / CPL) * 8 + l, kk = ks % CPL;
        const int g = c / CPG, cc = c % CPG;
        Wp[r * K + (size_t)(g * LPR + pl) * 8 + cc * CPL + kk] = W[i];
    }
}

int g_n_cu() {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    return n_cu;
}

} // namespace

// Lanes per row for an [N, K] matrix: long rows (few of them) spread over more
// lanes so the cohort's FMA chains use the whole chip; the 51866-row logits
// head packs 8 lanes per row and 2 rows per lane.
int fw_gemv16_lpr(int N, int K) {
    if (K % 64) return 0;
    if (N >= 16384) return 8;
    if (K >= 4096) return K % 256 == 0 ? 32 : K % 128 == 0 ? 16 : 8;
    return K % 128 == 0 ? 16 : 8;
}
bool fw_gemv16_ok(int N, int K) { return N > 0 && K > 0 && K % 64 == 0; }

void fw_launch_pack_gemv16(hipStream_t st, const uint16_t *W, uint16_t *Wp, int N, int K) {
    const size_t total = (size_t)N * K;
    size_t g = (total + 255) / 256;
    g = g < 65536 ? g : 65536;
    hipLaunchKernelGGL(k_pack_gemv16, dim3((unsigned)g), dim3(256), 0, st, W, Wp, N, K, fw_gemv16_lpr(N, K));
}

// per-tile argmax keys of the logits head: with keys the GEMV runs one row
// per lane and 4 waves, so a tile is (64 / lanes per row) * 4 rows
int fw_gemv16_key_blocks(int N, int K) {
    const int lpr = fw_gemv16_lpr(N, K);
    if (!lpr) return 0;
    const int rpt = 64 / lpr * 4;
    return (N + rpt - 1) / rpt;
}

namespace {

struct G16Args {
    const uint16_t *Wp;
    const float *bias, *x;
    float *y;
    int N, K, ns, ldy, mode;
    const float *gelu_tab, *lnw, *lnb;
    fwhip_filter filt;
    int use_filter;
    const int *initialp;
    unsigned long long *keys;
};

template <int LPR, int R, int SB, int WPB>
void g16_go(hipStream_t st, int grid, int nsg, const G16Args &a) {
    const size_t shm = (size_t)SB * a.K * 4;
    dim3 g(grid, nsg), b(64 * WPB);
#define G16_L(LN_, KEYS_)                                                                                          \
    hipLaunchKernelGGL((k_gemv16<LPR, R, SB, WPB, LN_, KEYS_>), g, b, shm, st, a.Wp, a.bias, a.x, a.y, a.N,        \
                       a.K, a.ns, a.ldy, a.mode, a.gelu_tab, a.lnw, a.lnb, a.filt, a.use_filter, a.initialp, a.keys)
    if (a.keys) {
        if constexpr (R == 1) { // the tiling fw_gemv16_key_blocks assumes
            if (a.lnw) G16_L(true, true);
            else G16_L(false, true);
        }
    } else if (a.lnw) {
        G16_L(true, false);
    } else {
        G16_L(false, false);
    }
#undef G16_L
}

// streams per block for a cohort of ns: the LDS copy of the rows must fit;
// the cohort splits into equal groups of at most sb_cap
int g16_pick_sb(int ns, int K, int sb_cap, int *nsg) {
    while (sb_cap > 1 && (size_t)sb_cap * K * 4 > 96 * 1024) sb_cap = (sb_cap + 1) / 2;
    int n = (ns + sb_cap - 1) / sb_cap;
    const int want = (ns + n - 1) / n;
    const int sb = want <= 1 ? 1 : want <= 2 ? 2 : want <= 4 ? 4 : want <= 5 ? 5 : want <= 8 ? 8 : want <= 10 ? 10
                 : want <= 12 ? 12 : 16;
    *nsg = (ns + sb - 1) / sb;
    return sb;
}

template <int LPR, int R, int WPB>
void g16_pipe(hipStream_t st, int grid_cap, int sb_cap, const G16Args &a) {
    constexpr int RPT = (64 / LPR) * R * WPB;
    const int ntile = (a.N + RPT - 1) / RPT;
    int nsg;
    const int sb = g16_pick_sb(a.ns, a.K, sb_cap, &nsg);
    const int grid = ntile < grid_cap ? ntile : grid_cap;
    switch (sb) {
    case 1: g16_go<LPR, R, 1, WPB>(st, grid, nsg, a); break;
    case 2: g16_go<LPR, R, 2, WPB>(st, grid, nsg, a); break;
    case 4: g16_go<LPR, R, 4, WPB>(st, grid, nsg, a); break;
    case 5: g16_go<LPR, R, 5, WPB>(st, grid, nsg, a); break;
    case 8: g16_go<LPR, R, 8, WPB>(st, grid, nsg, a); break;
    case 10: g16_go<LPR, R, 10, WPB>(st, grid, nsg, a); break;
    case 12: g16_go<LPR, R, 12, WPB>(st, grid, nsg, a); break;
    default: g16_go<LPR, R, 16, WPB>(st, grid, nsg, a); break;
    }
}

} // namespace

// y[s, :N] (mode 0 store, 1 add to y, 2 GELU) = W x_s + b for the ns rows of
// x [ns, K] (with lnw/lnb: LN(x_s), K <= 1280); W in slot order
// (fw_launch_pack_gemv16, lanes per row fw_gemv16_lpr(N, K)).  With keys (the
// logits head) the per-tile argmax keys [ns, fw_gemv16_key_blocks(N, K)] of the
// filtered row are written too.  r / sb_cap / grid_cap <= 0 take the tuned
// defaults for the shape.
void fw_launch_gemv16(hipStream_t st, const uint16_t *Wp, const float *bias, const float *x, float *y, int N, int K,
                      int ns, int ldy, int mode, const float *gelu_tab, const float *lnw, const float *lnb,
                      const fwhip_filter *filt, const int *initialp, unsigned long long *keys, int r, int sb_cap,
                      int grid_cap) {
    const int n_cu = g_n_cu();
    const int lpr = fw_gemv16_lpr(N, K);
    G16Args a{Wp, bias, x, y, N, K, ns, ldy, mode, gelu_tab, lnw, lnb, {}, filt != nullptr, initialp, keys};
    if (filt) a.filt = *filt;
    else memset(&a.filt, 0, sizeof a.filt);
    // shapes measured on MI355X for cohorts of 1, 10 and 16 streams:
    //  - the logits head (51866 rows): one row per lane, 10 streams a block
    //    (VALU-bound: ~1 FMA per weight element per stream), 2 blocks per CU,
    //    weights through the batch pipeline;
    //  - d x d (o, cross q/o): one stream per block, one row per lane (the
    //    most blocks; each re-reads the 3.3 MB matrix from L2 or the MALL);
    //  - q/k/v, fc1, fc2: 2 streams a block, 2 rows per lane; fc1 (N >= 4K)
    //    with 8 or more streams: 5 streams a block, one row per lane (10
    //    streams: step 413 -> 403 us; 16: 590 against 591; 4 streams keep the
    //    default: 353 against 354).
    const bool big = N >= 16384, small = N <= 1280 && K <= 1280, wide = !big && !small && N >= 4 * K && ns >= 8;
    if (r <= 0) r = big || small || ns == 1 || wide ? 1 : 2;
    if (sb_cap <= 0) sb_cap = big ? (ns >= 16 ? 5 : 10) : small ? 1 : wide ? 5 : 2;
    if (grid_cap <= 0) grid_cap = big ? (ns == 1 ? 4 * n_cu : ns >= 16 ? n_cu : 2 * n_cu) : 1 << 30;
    if (keys) r = 1; // the key layout (fw_gemv16_key_blocks) assumes one row per lane
#define G16_GO(L_, R_) g16_pipe<L_, R_, 4>(st, grid_cap, sb_cap, a)
    if (lpr == 8) {
        if (r >= 2) G16_GO(8, 2);
        else G16_GO(8, 1);
    } else if (lpr == 16) {
        if (r >= 2) G16_GO(16, 2);
        else G16_GO(16, 1);
    } else {
        if (r >= 2) G16_GO(32, 2);
        else G16_GO(32, 1);
    }
#undef G16_GO
}
