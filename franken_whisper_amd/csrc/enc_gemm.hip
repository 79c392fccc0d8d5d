// enc_gemm.hip — the encoder's dense contractions on MFMA (gfx950).
//
// One tiled GEMM template C[M,N] = A[M,K] x B[N,K]^T serves every encoder
// linear and the conv stem (as an im2col GEMM).  Operand kinds:
//   KIND_I8   : i8 x i8 -> i32 (v_mfma_i32_32x32x32_i8).  The int8 plan's
//               accumulators are exact integers, equal to the reference's
//               maddubs sum minus 128*colsum (nn.rs:1537-1771) or its i8 dot
//               (encoder.rs:2524-2606); epilogue ((f32)acc * s_x) * s_w (+ b)
//               in the reference's association (nn.rs:1660-1700,
//               encoder.rs:2573-2580).
//   KIND_F16S : f32 activations carried as an f16 pair (hi, lo = f16(a - hi))
//               against the f16 weights (exact: the reference dequantizes f16
//               weights to f32), two v_mfma_f32_32x32x16_f16 per product;
//               per-product error <= 2^-22 |a| + 2^-25, f32 accumulation.
//
// Block = 256 threads as 2x2 waves; block tile BM x BN (128x128 by default;
// 256x256 and 256x128 for sweeps);
// each wave owns (BM/2) x (BN/2) as a grid of 32x32 MFMA tiles.  K advances
// 64 bytes per stage (64 int8 or 32 f16 values); a stage is staged global ->
// registers -> LDS (rows padded to 80 bytes: conflict-free 16-byte reads),
// double buffered with one barrier per stage.  The epilogue is a template
// parameter so its loops fully unroll and the accumulators stay in registers.
//
// Tile order: the hardware deals blocks round-robin to the 8 XCDs; block ids
// are remapped so each XCD gets a contiguous run of tiles, walked in groups of
// 8 M-tiles (N outer), so an XCD's L2 holds the A rows of its group and one B
// tile at a time.
//
// MFMA operand layouts (gfx950): A lane l -> row l%32, k block (l/32)*16
// bytes; B lane l -> col l%32, same k block; accumulator r of lane l -> row
// (r/4)*8 + (l/32)*4 + r%4, col l%32.
#include <cstdlib>
#include <cstring>

#include "fw_enc.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define GEMM_LDSR 80 // LDS row stride in bytes (64 data + 16 pad)

__device__ __forceinline__ void fw_split2(float v, uint16_t &hi, uint16_t &lo) {
    asm volatile("" : "+v"(v));
    _Float16 h = (_Float16)v;
    float r = v - (float)h;
    asm volatile("" : "+v"(r));
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (_Float16)r);
}
// The same, or-ing into `of` whether the hi half overflows: |v| >= 65520
// rounds to an infinite f16 (65504 is the largest finite one), and the pair
// then carries inf / NaN instead of v.
__device__ __forceinline__ void fw_split2(float v, uint16_t &hi, uint16_t &lo, uint32_t &of) {
    of |= fabsf(v) >= 65520.0f ? 1u : 0u;
    fw_split2(v, hi, lo);
}

__global__ void __launch_bounds__(256) k_split_f16(const float4 *x, size_t n4, uint2 *hi, uint2 *lo, int *ovf) {
    uint32_t of = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
        const float4 v = x[i];
        uint16_t h[4], l[4];
        fw_split2(v.x, h[0], l[0], of);
        fw_split2(v.y, h[1], l[1], of);
        fw_split2(v.z, h[2], l[2], of);
        fw_split2(v.w, h[3], l[3], of);
        hi[i] = make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
        lo[i] = make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
    }
    if (of && ovf) *ovf = 1;
}

// n must be a multiple of 4 (rows of d, d % 128 == 0)
void fw_launch_split_f16(hipStream_t st, const float *x, size_t n, uint16_t *hi, uint16_t *lo, int *ovf) {
    const size_t n4 = n / 4;
    size_t g = (n4 + 255) / 256;
    g = g < 8192 ? g : 8192;
    hipLaunchKernelGGL(k_split_f16, dim3((unsigned)g), dim3(256), 0, st, (const float4 *)x, n4, (uint2 *)hi,
                       (uint2 *)lo, ovf);
}

// Epilogue for the 4 consecutive rows row0..row0+3 of one column.
template <int KIND, int EPI>
__device__ __forceinline__ void gemm_store4(const FwGemm &g, int row0, int col, const float (&a)[4]) {
    if (col >= g.N) return;
    if constexpr (EPI == FW_EPI_XKV) {
        const int d = g.ldc, l = col / (2 * d), r = col - l * 2 * d, kv = r >= d ? 1 : 0, c = r - kv * d;
        const int h = c >> 6, dd = c & 63;
        const float bias = g.bias ? g.bias[col] : 0.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int row = row0 + e;
            if (row >= g.M) continue;
            const int s = row / g.T, t = row - s * g.T;
            const size_t lh = ((size_t)s * g.L + l) * g.H + h;
            if (kv == 0) g.o16[0][(lh * g.T + t) * 64 + dd] = fw_f2h(a[e] * g.scale);
            else g.o16[1][(lh * 64 + dd) * g.T + t] = fw_f2h(a[e] + bias);
        }
        return;
    } else if constexpr (EPI == FW_EPI_QKV) {
        // head-major split outputs: Q, K as [B, H, T, 64]; V as [B, H, 64, Tp]
        const int d = g.ldc, which = col / d, cc = col - which * d, h = cc >> 6, dd = cc & 63;
        float bias = g.bias ? g.bias[col] : 0.0f;
        float sw = KIND == FW_KIND_I8 ? g.sw[col] : 1.0f;
        float v[4];
        uint16_t hi[4], lo[4];
        uint32_t of = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int row = row0 + e;
            float x = a[e];
            if constexpr (KIND == FW_KIND_I8) x = row < g.M ? x * g.sx[row] * sw : 0.0f;
            if (g.bias) x = x + bias;
            v[e] = x;
            fw_split2(v[e], hi[e], lo[e], of);
        }
        if (of && g.ovf) *g.ovf = 1;
        if (which < 2) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int row = row0 + e;
                if (row >= g.M) continue;
                int b = row / g.T, t = row - b * g.T;
                size_t o = (((size_t)b * g.H + h) * g.T + t) * 64 + dd;
                g.o16[2 * which][o] = hi[e];
                g.o16[2 * which + 1][o] = lo[e];
            }
        } else {
            // V^T key positions: bits 2 and 3 of the key index swapped within
            // each 16-key group (the attention kernel reads the 8 keys one MFMA
            // lane needs as one chunk); 4-key runs stay contiguous
            int b = row0 / g.T, t = row0 - b * g.T;
            size_t o = (((size_t)b * g.H + h) * 64 + dd) * g.Tp + fw_vt_pos(t);
            if ((t & 3) == 0 && t + 3 < g.T && row0 + 3 < g.M) {
                uint2 ph = make_uint2(hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16));
                uint2 pl = make_uint2(lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16));
                *(uint2 *)(g.o16[4] + o) = ph;
                *(uint2 *)(g.o16[5] + o) = pl;
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    int row = row0 + e;
                    if (row >= g.M) continue;
                    int bb = row / g.T, tt = row - bb * g.T;
                    size_t oo = (((size_t)bb * g.H + h) * 64 + dd) * g.Tp + fw_vt_pos(tt);
                    g.o16[4][oo] = hi[e];
                    g.o16[5][oo] = lo[e];
                }
            }
        }
        return;
    } else {
        float bias = g.bias ? g.bias[col] : 0.0f;
        float sw = (KIND == FW_KIND_I8 && EPI != FW_EPI_ACC32) ? g.sw[col] : 1.0f;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            int row = row0 + e;
            if (row >= g.M) continue;
            size_t o = (size_t)row * g.ldc + col;
            if constexpr (EPI == FW_EPI_ACC32) {
                if constexpr (KIND == FW_KIND_I8) ((int *)g.C)[o] = (int)a[e];
                else g.C[o] = a[e];
                continue;
            } else {
                float v = a[e];
                if constexpr (KIND == FW_KIND_I8) v = v * g.sx[row] * sw;
                if (g.bias) v = v + bias;
                if constexpr (EPI == FW_EPI_F32) {
                    g.C[o] = v;
                } else if constexpr (EPI == FW_EPI_RESID) {
                    g.C[o] = g.C[o] + v;
                } else if constexpr (EPI == FW_EPI_GELU_F32) {
                    g.C[o] = fw_gelu(v, g.gelu_tab);
                } else if constexpr (EPI == FW_EPI_GELU_SPLIT) {
                    uint16_t hi, lo;
                    uint32_t of = 0;
                    fw_split2(fw_gelu(v, g.gelu_tab), hi, lo, of);
                    if (of && g.ovf) *g.ovf = 1;
                    g.o16[0][o] = hi;
                    g.o16[1][o] = lo;
                } else if constexpr (EPI == FW_EPI_CONV2) {
                    int t = row % g.T;
                    g.C[o] = fw_gelu(v, g.gelu_tab) + g.pos[(size_t)t * g.ldc + col];
                }
            }
        }
    }
}

// Epilogue of a BM x BN block tile: wave (wm, wn) holds TM x TN 32x32
// accumulator tiles.  `lds` (>= 4 * 32 * 33 floats) is free scratch here.
// Block id -> tile sequence number.  map 1: the hardware deals blocks
// round-robin to the 8 XCDs, so block ids are remapped to give each XCD a
// contiguous run of the tile sequence; map 0: identity.
__device__ __forceinline__ int gemm_tile_order(int map) {
    const int nb = gridDim.x, bid = blockIdx.x;
    if (!map) return bid;
    const int xcd = bid & 7, loc = bid >> 3, per = nb >> 3, rem = nb & 7;
    return xcd < rem ? xcd * (per + 1) + loc : rem * (per + 1) + (xcd - rem) * per + loc;
}

template <int KIND, int EPI, int BM, int BN, typename accT>
__device__ __forceinline__ void gemm_epilogue(const FwGemm &g, accT (&acc)[BM / 64][BN / 64], unsigned char *lds,
                                              int m0, int n0) {
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    if constexpr (EPI == FW_EPI_QKV || EPI == FW_EPI_CONV2 || EPI == FW_EPI_XKV) {
        // Heavy epilogues: written once, in a runtime loop over this wave's
        // tiles, reading each tile back from a wave-private LDS slab (a fully
        // unrolled copy of such an epilogue per tile is too large to unroll,
        // which would push the accumulators to scratch memory).
        float *slab = (float *)lds + wave * (32 * 33);
        for (int tile = 0; tile < TM * TN; tile++) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    if (i * TN + j == tile)
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            slab[((r >> 2) * 8 + (lane >> 5) * 4 + (r & 3)) * 33 + (lane & 31)] = (float)acc[i][j][r];
            // the slab is private to this wave and a wave's LDS accesses run in
            // order: only the compiler must not reorder across this point
            asm volatile("" ::: "memory");
            const int i = tile / TN, j = tile - i * TN;
            const int col = n0 + wn * WN + j * 32 + (lane & 31);
            for (int q = 0; q < 4; q++) {
                const int rl = q * 8 + (lane >> 5) * 4;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = slab[(rl + e) * 33 + (lane & 31)];
                gemm_store4<KIND, EPI>(g, m0 + wm * WM + i * 32 + rl, col, v);
            }
            asm volatile("" ::: "memory");
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int col = n0 + wn * WN + j * 32 + (lane & 31);
            const int rb = m0 + wm * WM + i * 32 + (lane >> 5) * 4; // + q*8 + e
            if constexpr (KIND == FW_KIND_I8 && EPI == FW_EPI_ACC32) {
                // exact i32 accumulators: store the integers themselves
                if (col < g.N)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = rb + (r >> 2) * 8 + (r & 3);
                        if (row < g.M) ((int *)g.C)[(size_t)row * g.ldc + col] = acc[i][j][r];
                    }
            } else {
                // One 32x32 tile at a time: every load it needs (row scales,
                // residual values; rows clamped in bounds) is issued before the
                // first store, so the tile waits on memory once, not per element.
                const int colc = col < g.N ? col : g.N - 1;
                const float bias = g.bias ? g.bias[colc] : 0.0f;
                const float sw = KIND == FW_KIND_I8 ? g.sw[colc] : 1.0f;
                float sx[16], cv[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    int row = rb + (r >> 2) * 8 + (r & 3);
                    row = row < g.M ? row : g.M - 1;
                    if constexpr (KIND == FW_KIND_I8) sx[r] = g.sx[row];
                    if constexpr (EPI == FW_EPI_RESID) cv[r] = g.C[(size_t)row * g.ldc + colc];
                }
                if (col < g.N) {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = rb + (r >> 2) * 8 + (r & 3);
                        float v = (float)acc[i][j][r];
                        if constexpr (KIND == FW_KIND_I8) v = v * sx[r] * sw;
                        if (g.bias) v = v + bias;
                        if (row < g.M) {
                            const size_t o = (size_t)row * g.ldc + col;
                            if constexpr (EPI == FW_EPI_F32) {
                                g.C[o] = v;
                            } else if constexpr (EPI == FW_EPI_RESID) {
                                g.C[o] = cv[r] + v;
                            } else if constexpr (EPI == FW_EPI_GELU_F32) {
                                g.C[o] = fw_gelu(v, g.gelu_tab);
                            } else if constexpr (EPI == FW_EPI_GELU_SPLIT) {
                                uint16_t hi, lo;
                                uint32_t of = 0;
                                fw_split2(fw_gelu(v, g.gelu_tab), hi, lo, of);
                                if (of && g.ovf) *g.ovf = 1;
                                g.o16[0][o] = hi;
                                g.o16[1][o] = lo;
                            }
                        }
                    }
                }
            }
        }
}

template <int KIND, int EPI, int BM, int BN>
__global__ void __launch_bounds__(256) k_gemm(FwGemm g, int ntm, int ntn) {
    constexpr int NA = KIND == FW_KIND_F16S ? 2 : 1;
    constexpr int ES = KIND == FW_KIND_I8 ? 1 : 2;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int ROWS = NA * BM + BN; // LDS rows per stage
    constexpr int STAGE = ROWS * GEMM_LDSR;
    constexpr int CH = ROWS * 4 / 256; // 16-byte chunks per thread per stage
    constexpr int CHA = NA * BM / 64;  // chunks (per thread) that belong to A
    __shared__ __align__(16) unsigned char lds[2 * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-contiguous, M-grouped tile order
    const int t = gemm_tile_order(g.map);
    constexpr int GM = 8;
    const int gsize = GM * ntn, grp = t / gsize, first_m = grp * GM;
    const int gm = min(ntm - first_m, GM), rr = t - grp * gsize;
    const int m0 = (first_m + rr % gm) * BM, n0 = (rr / gm) * BN;
    const int nsteps = g.K * ES / 64;

    int4 stg[CH];
    auto gload = [&](int s) {
#pragma unroll
        for (int q = 0; q < CH; q++) {
            const int row = (tid >> 2) + q * 64, cc = tid & 3;
            const size_t koff = (size_t)s * 64 + cc * 16;
            if (q < CHA) {
                const int a = (q * 64) / BM, r = row - a * BM, gr = m0 + r;
                const unsigned char *base = (const unsigned char *)(a == 0 ? g.A : g.A2);
                stg[q] = gr < g.M ? *(const int4 *)(base + (size_t)gr * g.lda * ES + koff) : make_int4(0, 0, 0, 0);
            } else {
                const int gn = n0 + row - NA * BM;
                stg[q] = gn < g.N ? *(const int4 *)((const unsigned char *)g.B + (size_t)gn * g.ldb * ES + koff)
                                  : make_int4(0, 0, 0, 0);
            }
        }
    };
    auto lstore = [&](int buf) {
        unsigned char *base = lds + buf * STAGE;
#pragma unroll
        for (int q = 0; q < CH; q++) {
            const int row = (tid >> 2) + q * 64, cc = tid & 3;
            *(int4 *)(base + row * GEMM_LDSR + cc * 16) = stg[q];
        }
    };

    typedef typename std::conditional<KIND == FW_KIND_I8, v16i, v16f>::type accT;
    accT acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    gload(0);
    lstore(0);
    __syncthreads();
    int buf = 0;
    for (int s = 0; s < nsteps; s++) {
        if (s + 1 < nsteps) gload(s + 1);
        const unsigned char *tb = lds + buf * STAGE;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const int koff = ks * 32 + (lane >> 5) * 16;
            v4i af[NA][TM], bf[TN];
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int row = wm * WM + i * 32 + (lane & 31);
#pragma unroll
                for (int a = 0; a < NA; a++) af[a][i] = *(const v4i *)(tb + (a * BM + row) * GEMM_LDSR + koff);
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int row = wn * WN + j * 32 + (lane & 31);
                bf[j] = *(const v4i *)(tb + (NA * BM + row) * GEMM_LDSR + koff);
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    if constexpr (KIND == FW_KIND_I8) {
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0][i], bf[j], acc[i][j], 0, 0, 0);
                    } else {
                        const v8h bh = __builtin_bit_cast(v8h, bf[j]);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, af[0][i]), bh,
                                                                           acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, af[1][i]), bh,
                                                                           acc[i][j], 0, 0, 0);
                    }
                }
        }
        if (s + 1 < nsteps) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    gemm_epilogue<KIND, EPI, BM, BN>(g, acc, lds, m0, n0);
}

// ---------------------------------------------------------------------------
// Pipelined variant: operands go global -> LDS directly
// (global_load_lds_dwordx4, no staging registers), NS stages in flight, one
// barrier per stage.  LDS rows are 64 bytes with the 16-byte chunks of row r
// XOR-swizzled by (r ^ r>>2) & 3, so the MFMA fragment reads are free of bank
// conflicts.  Each wave loads ROWS/64 row groups of 16 rows per stage (one
// instruction writes 16 rows x 64 bytes = 1 KB contiguous in LDS).
__device__ __forceinline__ int gsw(int r) { return (r ^ (r >> 2)) & 3; }


template <int KIND, int EPI, int BM, int BN, int NS>
__global__ void __launch_bounds__(256) k_gemm2(FwGemm g, int ntm, int ntn) {
    constexpr int NA = KIND == FW_KIND_F16S ? 2 : 1;
    constexpr int ES = KIND == FW_KIND_I8 ? 1 : 2;
    constexpr int WM = BM / 2, WN = BN / 2, TM = WM / 32, TN = WN / 32;
    constexpr int ROWS = NA * BM + BN;
    constexpr int STAGE = ROWS * 64;
    constexpr int LPW = ROWS / 64; // load instructions per wave per stage
    __shared__ __align__(1024) unsigned char lds[NS * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    const int t = gemm_tile_order(g.map);
    constexpr int GM = 8;
    const int gsize = GM * ntn, grp = t / gsize, first_m = grp * GM;
    const int gm = min(ntm - first_m, GM), rr = t - grp * gsize;
    const int m0 = (first_m + rr % gm) * BM, n0 = (rr / gm) * BN;
    const int nsteps = g.K * ES / 64;

    // per-lane source rows of this wave's row groups (fixed over k)
    const unsigned char *src[LPW];
#pragma unroll
    for (int q = 0; q < LPW; q++) {
        const int lr = (wave * LPW + q) * 16 + (lane >> 2); // LDS row
        const int c = (lane & 3) ^ gsw(lr);                  // global chunk for this LDS slot
        if (lr < NA * BM) {
            const int a = lr / BM, r = lr - a * BM;
            int gr = m0 + r;
            gr = gr < g.M ? gr : g.M - 1; // rows past M: in-bounds reload, never stored
            src[q] = (const unsigned char *)(a == 0 ? g.A : g.A2) + (size_t)gr * g.lda * ES + c * 16;
        } else {
            int gn = n0 + lr - NA * BM;
            gn = gn < g.N ? gn : g.N - 1;
            src[q] = (const unsigned char *)g.B + (size_t)gn * g.ldb * ES + c * 16;
        }
    }
    auto issue = [&](int s) {
        const int sc = s < nsteps ? s : nsteps - 1; // past the end: harmless reload keeps vmcnt uniform
        unsigned char *dst = lds + (s % NS) * STAGE + wave * LPW * 1024;
#pragma unroll
        for (int q = 0; q < LPW; q++)
            __builtin_amdgcn_global_load_lds((const void *)(src[q] + (size_t)sc * 64),
                                             (void __attribute__((address_space(3))) *)(dst + q * 1024), 16, 0, 0);
    };

    typedef typename std::conditional<KIND == FW_KIND_I8, v16i, v16f>::type accT;
    accT acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // Fragment ping-pong: the two k-substeps (ks) of a stage use register
    // sets 0 and 1; the next substep's LDS reads are issued before the current
    // substep's MFMAs, so fragment latency hides behind MFMA issue.  The stage
    // barrier sits between the substeps of a stage.
    v4i fa[2][NA][TM], fb[2][TN];
    auto ldfrag = [&](int set, int stage, int ks) {
        const unsigned char *tb = lds + (stage % NS) * STAGE;
        const int c = ks * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int a = 0; a < NA; a++) {
                const int lr = a * BM + wm * WM + i * 32 + (lane & 31);
                fa[set][a][i] = *(const v4i *)(tb + lr * 64 + ((c ^ gsw(lr)) << 4));
            }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int lr = NA * BM + wn * WN + j * 32 + (lane & 31);
            fb[set][j] = *(const v4i *)(tb + lr * 64 + ((c ^ gsw(lr)) << 4));
        }
    };
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                if constexpr (KIND == FW_KIND_I8) {
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[set][0][i], fb[set][j], acc[i][j], 0, 0, 0);
                } else {
                    const v8h bh = __builtin_bit_cast(v8h, fb[set][j]);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, fa[set][0][i]), bh,
                                                                       acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, fa[set][1][i]), bh,
                                                                       acc[i][j], 0, 0, 0);
                }
            }
    };

#pragma unroll
    for (int p = 0; p < NS - 1; p++) issue(p);
    FW_WAIT_VM(LPW * (NS - 2)); // stage 0 landed
    asm volatile("s_barrier" ::: "memory");
    issue(NS - 1);
    ldfrag(0, 0, 0);
    for (int s = 0; s < nsteps; s++) {
        // set 0 was read a full MFMA block ago: completing it here is free and
        // lets the set-1 reads stay in flight under the set-0 MFMAs
        FW_WAIT_LGKM0();
        ldfrag(1, s, 1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(0);
        __builtin_amdgcn_sched_barrier(0);
        // stage s+1 visible to every wave; buffer (s % NS) is re-filled by
        // stage s+NS once every wave's reads of it have completed.  Run on the
        // last step too (a dummy stage, fragments never used): a branch here
        // would make the compiler wait on the new reads before the set-1 MFMAs.
        FW_WAIT_VM_LGKM0(LPW * (NS - 2));
        asm volatile("s_barrier" ::: "memory");
        issue(s + NS);
        ldfrag(0, s + 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(1);
        __builtin_amdgcn_sched_barrier(0);
    }
    FW_WAIT_VM(0);
    __syncthreads(); // LDS is reused by the heavy epilogues
    gemm_epilogue<KIND, EPI, BM, BN>(g, acc, lds, m0, n0);
}

// ---------------------------------------------------------------------------
// Persistent int8 GEMM.  One block per CU walks its share of the tile sequence
// through a single flattened (tile, k-step) pipeline: the operand stages of the
// next tile are already in flight while the current tile's epilogue runs, and
// its stores drain to memory under the next tile's MFMAs (a one-tile-per-block
// launch leaves every CU storing at once and the MFMAs idle meanwhile).
//
// Block = NW = WGM x WGN waves (2 per SIMD); block tile BM x BN, wave tile
// (BM/WGM) x (BN/WGN) of 32x32 i8 MFMA tiles; K advances 64 bytes per stage
// through an NS-stage global -> LDS ring (16-byte chunks XOR-swizzled by
// gsw(row)), one barrier per stage.
//
// vmcnt bookkeeping: stage s+1 is known to have landed once at most
// LPW*(NS-2) of this wave's loads are outstanding, which holds while every
// memory operation issued after stage s+1 is a load (loads return in order).
// Stores may complete out of order with loads, so before a tile's epilogue
// issues stores every outstanding load is waited for (vmcnt 0), and loads
// issued after the stores are the only ones later waits count on.
//
// The per-tile row scales sx, column scales sw and bias are staged into LDS
// with the tile's first stage (SCL 256-byte loads per wave, the same number
// for every wave so the counts above stay uniform; a tile's scales sit in the
// LDS half of its parity).
//
// Tile sequence: XCD x (blocks x, x+8, ...) owns a contiguous range of the
// GM=8-grouped tile order, walked by its blocks in lockstep, so the tiles in
// flight on one XCD share A row panels and B column panels in its L2.  With
// `wrows` > 0 (the QKV epilogue) M tiles never straddle a window of wrows rows:
// each window is tiled on its own, so every tile's rows share one window and
// start at a multiple of BM within it.
template <int EPI, int BM, int BN, int WGM, int WGN, int NS>
__global__ void __launch_bounds__(64 * WGM * WGN) k_gemm_pi8(FwGemm g, int ntm, int ntn, int ntw) {
    constexpr int NW = WGM * WGN, WM = BM / WGM, WN = BN / WGN, TM = WM / 32, TN = WN / 32;
    constexpr int STAGE = (BM + BN) * 64, LPW = STAGE / 1024 / NW;
    constexpr int SCL = (BM + 2 * BN + 64 * NW - 1) / (64 * NW); // scale loads per wave per tile
    constexpr int SCLN = SCL * NW * 64;                           // floats per parity
    constexpr bool QKV = EPI == FW_EPI_QKV;
    // wave-private LDS slab: QKV turns 32 x 32 f32 tiles (rows of 40), the
    // index epilogue sends 32 x WN u16 tiles out as whole rows
    constexpr int SLABB = QKV ? 32 * 40 * 4 : (EPI == FW_EPI_F16IDX ? 32 * WN * 2 : 0); // bytes per wave
    static_assert(STAGE % (1024 * NW) == 0, "stage loads must split evenly over waves");
    __shared__ __align__(1024) unsigned char lds[NS * STAGE + 2 * SCLN * 4 + NW * SLABB];
    float *scl = (float *)(lds + NS * STAGE);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    const int G = gridDim.x, xcd = blockIdx.x & 7, loc = blockIdx.x >> 3, nloc = G >> 3;
    const int ntiles = ntm * ntn;
    const int xs = (int)((long long)ntiles * xcd / 8), xe = (int)((long long)ntiles * (xcd + 1) / 8);
    const int my_n = xe - xs > loc ? (xe - xs - loc + nloc - 1) / nloc : 0;
    const int nsteps = g.K / 64;
    const int total = my_n * nsteps;
    if (total == 0) return;
    uint32_t ovf_any = 0; // an f16-pair value past the f16 range (FW_EPI_QKV)
    // tile ti of this block -> first row, valid rows, first column
    auto coords = [&](int ti, int &m0, int &mrows, int &n0) {
        const int t = xs + loc + ti * nloc;
        constexpr int GM = 8;
        const int gsize = GM * ntn, grp = t / gsize, first_m = grp * GM;
        const int gm = min(ntm - first_m, GM), rr = t - grp * gsize;
        const int mt = first_m + rr % gm;
        n0 = (rr / gm) * BN;
        if (ntw > 0) {
            const int w = mt / ntw, tt = mt - w * ntw;
            m0 = w * g.T + tt * BM;
            mrows = min(BM, g.T - tt * BM);
        } else {
            m0 = mt * BM;
            mrows = min(BM, g.M - m0);
        }
    };
    // issue side: tile and step of the next stage to load, per-lane sources
    int it_tile = 0, it_step = 0;
    const unsigned char *src[LPW];
    const float *ssrc[SCL];
    auto set_src = [&](int ti) {
        int m0, mrows, n0;
        coords(ti, m0, mrows, n0);
#pragma unroll
        for (int q = 0; q < LPW; q++) {
            const int lr = (wave * LPW + q) * 16 + (lane >> 2);
            const int c = (lane & 3) ^ gsw(lr);
            if (lr < BM)
                src[q] = (const unsigned char *)g.A + (size_t)(m0 + min(lr, mrows - 1)) * g.lda + c * 16;
            else
                src[q] = (const unsigned char *)g.B + (size_t)min(n0 + lr - BM, g.N - 1) * g.ldb + c * 16;
        }
#pragma unroll
        for (int q = 0; q < SCL; q++) {
            const int e = (q * NW + wave) * 64 + lane;
            if (e < BM) ssrc[q] = g.sx + m0 + min(e, mrows - 1);
            else if (e < BM + BN) ssrc[q] = g.sw + min(n0 + e - BM, g.N - 1);
            else ssrc[q] = (g.bias ? g.bias : g.sw) + min(n0 + max(e - BM - BN, 0), g.N - 1);
        }
    };
    set_src(0);
    auto issue = [&](int gs) {
        unsigned char *dst = lds + (gs % NS) * STAGE + wave * LPW * 1024;
        const int sc = it_tile < my_n ? it_step : nsteps - 1; // past the last tile: in-bounds reload
#pragma unroll
        for (int q = 0; q < LPW; q++)
            __builtin_amdgcn_global_load_lds((const void *)(src[q] + (size_t)sc * 64),
                                             (void __attribute__((address_space(3))) *)(dst + q * 1024), 16, 0, 0);
        if (it_step == 0) {
            float *sd = scl + (it_tile & 1) * SCLN + wave * 64;
#pragma unroll
            for (int q = 0; q < SCL; q++)
                __builtin_amdgcn_global_load_lds((const void *)ssrc[q],
                                                 (void __attribute__((address_space(3))) *)(sd + q * NW * 64), 4,
                                                 0, 0);
        }
        if (++it_step == nsteps) {
            if (it_tile < my_n) {
                it_step = 0;
                if (++it_tile < my_n) set_src(it_tile);
            } else {
                it_step = nsteps - 1;
            }
        }
    };

    v16i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
    v4i fa[2][TM], fb[2][TN];
    auto ldfrag = [&](int set, int stage, int ks) {
        const unsigned char *tb = lds + (stage % NS) * STAGE;
        const int c = ks * 2 + (lane >> 5);
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int lr = wm * WM + i * 32 + (lane & 31);
            fa[set][i] = *(const v4i *)(tb + lr * 64 + ((c ^ gsw(lr)) << 4));
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            const int lr = BM + wn * WN + j * 32 + (lane & 31);
            fb[set][j] = *(const v4i *)(tb + lr * 64 + ((c ^ gsw(lr)) << 4));
        }
    };
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
    };

#pragma unroll
    for (int p = 0; p < NS - 1; p++) issue(p);
    FW_WAIT_VM(0);
    asm volatile("s_barrier" ::: "memory");
    issue(NS - 1);
    ldfrag(0, 0, 0);
    const bool has_bias = g.bias != nullptr;
    int tile = 0, s = 0;
    for (int gs = 0; gs < total; gs++) {
        FW_WAIT_LGKM0();
        ldfrag(1, gs, 1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(0);
        __builtin_amdgcn_sched_barrier(0);
        FW_WAIT_VM_LGKM0(LPW * (NS - 2));
        asm volatile("s_barrier" ::: "memory");
        const bool last = s == nsteps - 1;
        if (!last) issue(gs + NS);
        ldfrag(0, gs + 1, 0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(1);
        __builtin_amdgcn_sched_barrier(0);
        if (!last) {
            s++;
            continue;
        }
        // ---- epilogue of this block's tile `tile` ----
        FW_WAIT_VM(0);
        int m0, mrows, n0;
        coords(tile, m0, mrows, n0);
        // lane-derived offsets recomputed here from an opaque copy of the lane
        // id, so per-element addresses are not hoisted out of the tile loop
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const float *ssx = scl + (tile & 1) * SCLN, *ssw = ssx + BM, *sbi = ssw + BN;
        // A 32 x WN u16 tile (accumulator layout: element r of lane l is row
        // (r/4)*8 + (l/32)*4 + r%4, column j*32 + l%32), put into this wave's
        // slab one 32-column tile j at a time, then flushed to rows dst + row*ld,
        // row < vrows, as 16-byte runs of whole rows (WN/8 lanes per row).  The
        // slab is private to the wave and a wave's LDS accesses run in order:
        // only the compiler must not reorder them.
        uint16_t *const sl = (uint16_t *)(lds + NS * STAGE + 2 * SCLN * 4 + wave * SLABB);
        auto slab_put = [&](int j, const uint16_t (&u)[16]) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int r = 0; r < 16; r++) sl[((r >> 2) * 8 + (ln >> 5) * 4 + (r & 3)) * WN + j * 32 + (ln & 31)] = u[r];
            asm volatile("" ::: "memory");
        };
        auto slab_flush = [&](uint16_t *dst, size_t ld, int vrows) {
            constexpr int LPR = WN / 8, RPI = 64 / LPR;
            asm volatile("" ::: "memory");
#pragma unroll
            for (int q = 0; q < 32 / RPI; q++) {
                const int row = q * RPI + ln / LPR, ch = ln % LPR;
                const uint4 w = *(const uint4 *)(sl + row * WN + ch * 8);
                if (row < vrows) *(uint4 *)(dst + row * ld + ch * 8) = w;
            }
            asm volatile("" ::: "memory");
        };
        // Full-line f32 results (two 128-byte rows per store) are written
        // non-temporally: they are not read again by this kernel and would only
        // evict operand panels from L2.  The QKV epilogue's 16-byte runs stay
        // cached so L2 can merge them into lines (non-temporal partial lines
        // measured 1.6x slower).
        if constexpr (EPI == FW_EPI_RESID) {
            static_assert(TM * TN <= 4, "residual values of the wave tile are held in registers");
            // residual values of every element first: one wait, then the stores
            float cv[TM][TN][16];
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int col = min(n0 + wn * WN + j * 32 + (ln & 31), g.N - 1);
                    const int rl = wm * WM + i * 32 + (ln >> 5) * 4;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = m0 + min(rl + (r >> 2) * 8 + (r & 3), mrows - 1);
                        cv[i][j][r] = g.C[(size_t)row * g.ldc + col];
                    }
                }
            FW_WAIT_VM(0);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int cl = wn * WN + j * 32 + (ln & 31), col = n0 + cl;
                    const int rl = wm * WM + i * 32 + (ln >> 5) * 4;
                    const float s2 = ssw[cl], bb = sbi[cl];
                    v4f sr[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) sr[q] = *(const v4f *)(ssx + rl + q * 8);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int rw = rl + (r >> 2) * 8 + (r & 3);
                        float v = (float)acc[i][j][r] * sr[r >> 2][r & 3] * s2;
                        if (has_bias) v = v + bb;
                        if (rw < mrows && col < g.N) __builtin_nontemporal_store(cv[i][j][r] + v, g.C + (size_t)(m0 + rw) * g.ldc + col);
                    }
                }
        } else if constexpr (EPI == FW_EPI_F16IDX) {
            const bool wide = n0 + BN <= g.N;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int r0 = wm * WM + i * 32, vrows = mrows - r0;
                uint16_t u[TN][16];
                bool sent = false;
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int cl = wn * WN + j * 32 + (ln & 31);
                    const int rl = r0 + (ln >> 5) * 4;
                    const float s2 = ssw[cl], bb = sbi[cl];
                    v4f sr[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) sr[q] = *(const v4f *)(ssx + rl + q * 8);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        float v = (float)acc[i][j][r] * sr[r >> 2][r & 3] * s2;
                        if (has_bias) v = v + bb;
                        const bool in = fabsf(v) < FW_GIDX_LIM;
                        u[j][r] = in ? fw_f2h(v) : (uint16_t)FW_GIDX_SENT;
                        sent |= !in;
                        acc[i][j][r] = __float_as_int(v); // kept for the rare side stores
                    }
                }
                if (__builtin_amdgcn_ballot_w64(sent)) {
                    // values beyond the table's range: exact f32 into the side array
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int rw = r0 + (r >> 2) * 8 + (ln >> 5) * 4 + (r & 3);
                            const int col = n0 + wn * WN + j * 32 + (ln & 31);
                            if (u[j][r] == (uint16_t)FW_GIDX_SENT && rw < mrows && col < g.N)
                                g.C[(size_t)(m0 + rw) * g.ldc + col] = __int_as_float(acc[i][j][r]);
                        }
                }
                if (vrows <= 0) continue;
                if (wide) {
#pragma unroll
                    for (int j = 0; j < TN; j++) slab_put(j, u[j]);
                    slab_flush(g.o16[0] + (size_t)(m0 + r0) * g.ldc + n0 + wn * WN, g.ldc, vrows);
                } else {
#pragma unroll
                    for (int j = 0; j < TN; j++)
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int rw = (r >> 2) * 8 + (ln >> 5) * 4 + (r & 3);
                            const int col = n0 + wn * WN + j * 32 + (ln & 31);
                            if (rw < vrows && col < g.N) g.o16[0][(size_t)(m0 + r0 + rw) * g.ldc + col] = u[j][r];
                        }
                }
            }
        } else if constexpr (EPI == FW_EPI_F32 || EPI == FW_EPI_ACC32) {
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int cl = wn * WN + j * 32 + (ln & 31), col = n0 + cl;
                    const int rl = wm * WM + i * 32 + (ln >> 5) * 4;
                    const float s2 = ssw[cl], bb = sbi[cl];
                    v4f sr[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) sr[q] = *(const v4f *)(ssx + rl + q * 8);
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int rw = rl + (r >> 2) * 8 + (r & 3);
                        if (rw < mrows && col < g.N) {
                            const size_t o = (size_t)(m0 + rw) * g.ldc + col;
                            if constexpr (EPI == FW_EPI_ACC32) {
                                ((int *)g.C)[o] = acc[i][j][r];
                            } else {
                                float v = (float)acc[i][j][r] * sr[r >> 2][r & 3] * s2;
                                if (has_bias) v = v + bb;
                                __builtin_nontemporal_store(v, g.C + o);
                            }
                        }
                    }
                }
        } else if constexpr (QKV) {
            // Q, K: [B, H, T, 64] f16 hi/lo rows, written through a wave-private
            // LDS slab so each lane stores 16 consecutive dims (32-byte runs).
            // V^T: [B, H, 64, Tp] at key positions fw_vt_pos(t); a lane's 8
            // values r = 8c .. 8c+7 sit at 8 consecutive positions (window
            // tiles start at multiples of 32), so they go out as 16-byte runs.
            float *slab = (float *)(lds + NS * STAGE + 2 * SCLN * 4 + wave * SLABB);
            const int d = g.ldc, wnd = m0 / g.T, tb0 = m0 - wnd * g.T;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    const int c0 = n0 + wn * WN + j * 32; // 32 columns of one head
                    const int cl = c0 - n0 + (ln & 31), col = n0 + cl;
                    const int rl = wm * WM + i * 32 + (ln >> 5) * 4;
                    const float s2 = ssw[cl], bb = sbi[cl];
                    v4f sr[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) sr[q] = *(const v4f *)(ssx + rl + q * 8);
                    float v[16];
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        v[r] = (float)acc[i][j][r] * sr[r >> 2][r & 3] * s2;
                        if (has_bias) v[r] = v[r] + bb;
                    }
                    if (c0 >= g.N) continue;
                    const int which = c0 / d, cc = c0 - which * d, h = cc >> 6, dd0 = cc & 63;
                    const int t0 = tb0 + wm * WM + i * 32; // window position of the tile's first row
                    const int vrows = mrows - (wm * WM + i * 32);
                    if (vrows <= 0) continue;
                    if (which == 2) {
                        const int dd = dd0 + (ln & 31);
                        uint16_t *vh = g.o16[4] + (((size_t)wnd * g.H + h) * 64 + dd) * g.Tp;
                        uint16_t *vl = g.o16[5] + (((size_t)wnd * g.H + h) * 64 + dd) * g.Tp;
#pragma unroll
                        for (int c = 0; c < 2; c++) {
                            const int pb = t0 + 16 * c + 8 * (ln >> 5); // first of 8 positions
                            uint16_t hi[8], lo[8];
#pragma unroll
                            for (int e = 0; e < 8; e++) fw_split2(v[8 * c + e], hi[e], lo[e], ovf_any);
                            if (16 * c + 16 <= vrows) {
                                uint4 ph, pl;
                                ph.x = hi[0] | ((uint32_t)hi[1] << 16);
                                ph.y = hi[2] | ((uint32_t)hi[3] << 16);
                                ph.z = hi[4] | ((uint32_t)hi[5] << 16);
                                ph.w = hi[6] | ((uint32_t)hi[7] << 16);
                                pl.x = lo[0] | ((uint32_t)lo[1] << 16);
                                pl.y = lo[2] | ((uint32_t)lo[3] << 16);
                                pl.z = lo[4] | ((uint32_t)lo[5] << 16);
                                pl.w = lo[6] | ((uint32_t)lo[7] << 16);
                                *(uint4 *)(vh + pb) = ph;
                                *(uint4 *)(vl + pb) = pl;
                            } else {
#pragma unroll
                                for (int e = 0; e < 8; e++) {
                                    // value e is key t0 + 16c + 8*(e/4) + 4*(lane/32) + e%4
                                    const int rr = 16 * c + 8 * (e >> 2) + 4 * (ln >> 5) + (e & 3);
                                    if (rr < vrows) {
                                        const int p = fw_vt_pos(t0 + rr);
                                        vh[p] = hi[e];
                                        vl[p] = lo[e];
                                    }
                                }
                            }
                        }
                    } else {
                        // the slab is private to this wave and a wave's LDS accesses
                        // run in order: only the compiler must not reorder them
                        asm volatile("" ::: "memory");
#pragma unroll
                        for (int r = 0; r < 16; r++)
                            slab[((r >> 2) * 8 + (ln >> 5) * 4 + (r & 3)) * 40 + (ln & 31)] = v[r];
                        asm volatile("" ::: "memory");
                        const int row = ln >> 1, half = ln & 1;
                        v4f w4[4];
#pragma unroll
                        for (int q = 0; q < 4; q++) w4[q] = *(const v4f *)(slab + row * 40 + half * 16 + q * 4);
                        asm volatile("" ::: "memory");
                        if (row < vrows) {
                            uint32_t ph[8], pl[8];
#pragma unroll
                            for (int q = 0; q < 8; q++) {
                                uint16_t h0, l0, h1, l1;
                                fw_split2(w4[q >> 1][(q & 1) * 2], h0, l0, ovf_any);
                                fw_split2(w4[q >> 1][(q & 1) * 2 + 1], h1, l1, ovf_any);
                                ph[q] = h0 | ((uint32_t)h1 << 16);
                                pl[q] = l0 | ((uint32_t)l1 << 16);
                            }
                            const size_t o = (((size_t)wnd * g.H + h) * g.T + t0 + row) * 64 + dd0 + half * 16;
                            uint4 *qh = (uint4 *)(g.o16[2 * which] + o), *ql = (uint4 *)(g.o16[2 * which + 1] + o);
                            qh[0] = make_uint4(ph[0], ph[1], ph[2], ph[3]);
                            qh[1] = make_uint4(ph[4], ph[5], ph[6], ph[7]);
                            ql[0] = make_uint4(pl[0], pl[1], pl[2], pl[3]);
                            ql[1] = make_uint4(pl[4], pl[5], pl[6], pl[7]);
                        }
                    }
                }
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
        issue(gs + NS);
        tile++;
        s = 0;
    }
    FW_WAIT_VM(0);
    if constexpr (EPI == FW_EPI_QKV)
        if (ovf_any && g.ovf) *g.ovf = 1;
}

// ---------------------------------------------------------------------------
// Tile choice: register-staged tiles (r256x256, r256x128, r128x128) and the
// pipelined direct-to-LDS tiles (p256x256, p256x128, p128x128 with 4 stages,
// or 2-3 stages: n2, n3).  FWHIP_GEMM_TILE=<name> forces one (tuning sweeps).
static const char *kTileNames[9] = {"r256x256", "r256x128", "r128x128", "p256x256", "p256x128",
                                    "p128x128", "p256x128n2", "p128x128n3", "p128x128n2"};

static int forced_tile() {
    static int forced = -2;
    if (forced == -2) {
        forced = -1;
        const char *e = getenv("FWHIP_GEMM_TILE");
        if (e)
            for (int i = 0; i < 9; i++)
                if (!strcmp(e, kTileNames[i])) forced = i;
    }
    return forced;
}

// Measured (large-v3-turbo int8 plan, 10 windows): p128x128 with 3 stages
// (three blocks per CU, so one block's epilogue overlaps the others' MFMAs)
// 885 TOP/s over the encoder's GEMMs, ahead of every other variant
// (p128x128n2 816, p128x128 851, p256x128n2 722, p256x256 640).
static int pick_tile(int M, int N, int ncu) {
    int f = forced_tile();
    if (f >= 0) return f;
    (void)M;
    (void)N;
    (void)ncu;
    return 7;
}

template <int KIND, int EPI, int BM, int BN>
static void launch_one(hipStream_t st, const FwGemm &g) {
    int ntm = (g.M + BM - 1) / BM, ntn = (g.N + BN - 1) / BN;
    hipLaunchKernelGGL((k_gemm<KIND, EPI, BM, BN>), dim3(ntm * ntn), dim3(256), 0, st, g, ntm, ntn);
}

template <int KIND, int EPI, int BM, int BN, int NS>
static void launch_pipe(hipStream_t st, const FwGemm &g) {
    int ntm = (g.M + BM - 1) / BM, ntn = (g.N + BN - 1) / BN;
    hipLaunchKernelGGL((k_gemm2<KIND, EPI, BM, BN, NS>), dim3(ntm * ntn), dim3(256), 0, st, g, ntm, ntn);
}

template <int KIND, int EPI>
static void launch_tiles(hipStream_t st, const FwGemm &g, int tile) {
    constexpr int NSB = KIND == FW_KIND_I8 ? 4 : 3; // stages of the 256-row pipelined tiles (LDS <= 160 KB)
    switch (tile) {
    case 0: launch_one<KIND, EPI, 256, 256>(st, g); break;
    case 1: launch_one<KIND, EPI, 256, 128>(st, g); break;
    case 2: launch_one<KIND, EPI, 128, 128>(st, g); break;
    case 3: launch_pipe<KIND, EPI, 256, 256, NSB>(st, g); break;
    case 4: launch_pipe<KIND, EPI, 256, 128, NSB>(st, g); break;
    case 5: launch_pipe<KIND, EPI, 128, 128, 4>(st, g); break;
    case 6: launch_pipe<KIND, EPI, 256, 128, 2>(st, g); break;
    case 7: launch_pipe<KIND, EPI, 128, 128, 3>(st, g); break;
    default: launch_pipe<KIND, EPI, 128, 128, 2>(st, g); break;
    }
}

// Persistent int8 launch: 256x256 tiles (8 waves of 128x64) for wide outputs,
// 256x128 (8 waves of 64x64) for N < 2048 and for the residual epilogue, whose
// wave tile must fit its residual values in registers.  One block per CU
// (LDS and registers admit no second); the grid is a multiple of 8 so block
// b runs on XCD b % 8.
template <int EPI, int BM, int BN, int WGM, int WGN>
static void launch_pi8(hipStream_t st, const FwGemm &g, int ncu) {
    int ntw = 0, ntm;
    if (EPI == FW_EPI_QKV) {
        ntw = (g.T + BM - 1) / BM;
        ntm = (g.M / g.T) * ntw;
    } else {
        ntm = (g.M + BM - 1) / BM;
    }
    const int ntn = (g.N + BN - 1) / BN;
    const int grid = ncu >= 8 ? ncu / 8 * 8 : 8;
    hipLaunchKernelGGL((k_gemm_pi8<EPI, BM, BN, WGM, WGN, 3>), dim3(grid), dim3(64 * WGM * WGN), 0, st, g, ntm, ntn,
                       ntw);
}

template <int EPI>
static void launch_pi8_tiles(hipStream_t st, const FwGemm &g, int ncu) {
    if constexpr (EPI != FW_EPI_RESID)
        if (g.N >= 2048) {
            launch_pi8<EPI, 256, 256, 2, 4>(st, g, ncu);
            return;
        }
    launch_pi8<EPI, 256, 128, 4, 2>(st, g, ncu);
}

bool fw_launch_gemm(hipStream_t st, int kind, const FwGemm &g0) {
    static int map = -1;
    if (map < 0) {
        const char *e = getenv("FWHIP_GEMM_MAP");
        map = e ? atoi(e) : 1;
    }
    FwGemm g = g0;
    g.map = map;
    static int ncu = 0;
    if (!ncu) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
        if (ncu <= 0) ncu = 256;
    }
    static int pi8 = -1;
    if (pi8 < 0) {
        const char *e = getenv("FWHIP_GEMM_I8P");
        pi8 = e ? atoi(e) : 1;
    }
    // One window (M <= 1536 rows) fills the CUs better with the one-tile-per-
    // block kernels' tiles: the persistent kernel's 256 x 256 tiles give the
    // q/k/v GEMM 90 tiles for 256 CUs (one-window encoder pass 8.35 -> 7.78
    // ms; from two windows on the persistent kernel is faster: 9.81 against
    // 10.15 ms, ten 36.1 against 40.3).  Both routes give the same bits.
    if (kind == FW_KIND_I8 && pi8 && g.M > 1536 && g.K % 64 == 0 &&
        (g.epi != FW_EPI_QKV || (g.T > 0 && g.M % g.T == 0))) {
        switch (g.epi) {
        case FW_EPI_F32: launch_pi8_tiles<FW_EPI_F32>(st, g, ncu); return true;
        case FW_EPI_RESID: launch_pi8_tiles<FW_EPI_RESID>(st, g, ncu); return true;
        case FW_EPI_QKV: launch_pi8_tiles<FW_EPI_QKV>(st, g, ncu); return true;
        case FW_EPI_ACC32: launch_pi8_tiles<FW_EPI_ACC32>(st, g, ncu); return true;
        case FW_EPI_F16IDX: launch_pi8_tiles<FW_EPI_F16IDX>(st, g, ncu); return true;
        default: break;
        }
    }
    int tile = pick_tile(g.M, g.N, ncu);
    if (kind == FW_KIND_I8) {
        switch (g.epi) {
        case FW_EPI_F32: launch_tiles<FW_KIND_I8, FW_EPI_F32>(st, g, tile); return true;
        case FW_EPI_RESID: launch_tiles<FW_KIND_I8, FW_EPI_RESID>(st, g, tile); return true;
        case FW_EPI_QKV: launch_tiles<FW_KIND_I8, FW_EPI_QKV>(st, g, tile); return true;
        case FW_EPI_ACC32: launch_tiles<FW_KIND_I8, FW_EPI_ACC32>(st, g, tile); return true;
        default: return false;
        }
    } else {
        switch (g.epi) {
        case FW_EPI_F32: launch_tiles<FW_KIND_F16S, FW_EPI_F32>(st, g, tile); return true;
        case FW_EPI_RESID: launch_tiles<FW_KIND_F16S, FW_EPI_RESID>(st, g, tile); return true;
        case FW_EPI_GELU_F32: launch_tiles<FW_KIND_F16S, FW_EPI_GELU_F32>(st, g, tile); return true;
        case FW_EPI_GELU_SPLIT: launch_tiles<FW_KIND_F16S, FW_EPI_GELU_SPLIT>(st, g, tile); return true;
        case FW_EPI_CONV2: launch_tiles<FW_KIND_F16S, FW_EPI_CONV2>(st, g, tile); return true;
        case FW_EPI_QKV: launch_tiles<FW_KIND_F16S, FW_EPI_QKV>(st, g, tile); return true;
        case FW_EPI_XKV: launch_tiles<FW_KIND_F16S, FW_EPI_XKV>(st, g, tile); return true;
        default: return false;
        }
    }
}
