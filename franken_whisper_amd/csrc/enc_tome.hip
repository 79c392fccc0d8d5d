// enc_tome.hip — ToMe token merging for the batched encoder (gfx950):
// tome_merge / tome_unmerge (encoder.rs:1403-1517) per 30 s window, in the
// strict-parity arithmetic the reference uses with FT_SGEMM_STRICT_PARITY=1,
// so merge decisions and merged rows are bit-identical to it given the same
// encoder rows:
//  - A = rows 0, 2, 4, ..., B = rows 1, 3, ... of each window;
//  - sim[a][b] = ascending-k sequential f32 sum of products (nn::matmul's
//    strict path, nn.rs:587-604) — a 64 x 64 tile per block, each thread 4 x 4
//    outputs with separate multiply and add (no FMA), K staged in LDS;
//  - row norms: sqrt of the sequential f32 sum of v*v, floored at 1e-9;
//  - cos = sim / (na * nb); per A row the first strict maximum over B (one
//    ordered key per tile: value first, then the lower index);
//  - a stable descending ranking of the best similarities (ties keep the lower
//    A index); the r best A rows merge into their B partner;
//  - a merged B row is its B row plus the merged A rows in ascending A order,
//    divided by the count when the count exceeds one; then the kept A rows in
//    ascending order; umap maps every original row to its merged row.
#include <cmath>

#include "fw_dec.h"
#include "fw_enc.h"

namespace {

constexpr int TM_TILE = 64, TM_KC = 32, TM_LD = TM_TILE + 4;

// sequential f32 sum of squares of a row, sqrt, floor 1e-9 (f32::max)
__global__ void __launch_bounds__(256) k_tome_norm(const float *x, int rows, int d, float *nrm) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= rows) return;
    const float4 *p = (const float4 *)(x + (size_t)r * d);
    float s = 0.0f;
    for (int i = 0; i < (d >> 2); i++) {
        const float4 v = p[i];
        s = s + v.x * v.x;
        s = s + v.y * v.y;
        s = s + v.z * v.z;
        s = s + v.w * v.w;
    }
    s = sqrtf(s);
    nrm[r] = s > 1e-9f ? s : 1e-9f;
}

// keys[((w * n_a + a) * nbt + bt)] = max over the tile's b of the ordered key
// (cos, b); 0 when no cos in the tile exceeds -inf
__global__ void __launch_bounds__(256) k_tome_sim(const float *x, const float *nrm, int T, int d, int n_a, int n_b,
                                                  int nbt, unsigned long long *keys) {
    __shared__ __align__(16) float As[TM_KC][TM_LD], Bs[TM_KC][TM_LD];
    const int bt = blockIdx.x, at = blockIdx.y, w = blockIdx.z, t = threadIdx.x;
    const int tx = t & 15, ty = t >> 4;
    const int a0 = at * TM_TILE, b0 = bt * TM_TILE;
    const float *xw = x + (size_t)w * T * d;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < d; k0 += TM_KC) {
        // 64 rows x 32 columns of A and of B: two float4 of each per thread
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int i = t + u * 256, row = i >> 3, c4 = i & 7;
            const int a = a0 + row, b = b0 + row;
            const float4 va = ((const float4 *)(xw + (size_t)(2 * (a < n_a ? a : n_a - 1)) * d + k0))[c4];
            const float4 vb = ((const float4 *)(xw + (size_t)(2 * (b < n_b ? b : n_b - 1) + 1) * d + k0))[c4];
            As[c4 * 4 + 0][row] = va.x;
            As[c4 * 4 + 1][row] = va.y;
            As[c4 * 4 + 2][row] = va.z;
            As[c4 * 4 + 3][row] = va.w;
            Bs[c4 * 4 + 0][row] = vb.x;
            Bs[c4 * 4 + 1][row] = vb.y;
            Bs[c4 * 4 + 2][row] = vb.z;
            Bs[c4 * 4 + 3][row] = vb.w;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < TM_KC; k++) {
            const float4 av = *(const float4 *)&As[k][ty * 4];
            const float4 bv = *(const float4 *)&Bs[k][tx * 4];
            const float ar[4] = {av.x, av.y, av.z, av.w}, br[4] = {bv.x, bv.y, bv.z, bv.w};
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++) acc[i][j] = acc[i][j] + ar[i] * br[j];
        }
        __syncthreads();
    }
    const float *nw = nrm + (size_t)w * T;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int a = a0 + ty * 4 + i;
        const float na = nw[2 * (a < n_a ? a : n_a - 1)];
        unsigned long long km = 0ull;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int b = b0 + tx * 4 + j;
            if (b < n_b) {
                const float c = acc[i][j] / (na * nw[2 * b + 1]);
                const unsigned long long kv = am_key(c, b);
                km = kv > km ? kv : km;
            }
        }
        km = row16_max_u64(km); // the 16 threads of this a (lanes 16 * (ty % 4) ..)
        if (tx == 0 && a < n_a) keys[((size_t)w * n_a + a) * nbt + bt] = km;
    }
}

__device__ __forceinline__ float tm_key_value(unsigned long long k) {
    const uint32_t u = (uint32_t)(k >> 32);
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

// one block per window: best edges, the stable ranking, merge lists, kept
// rows and the unmerge map
__global__ void __launch_bounds__(1024) k_tome_select(const unsigned long long *keys, int T, int n_a, int n_b, int nbt,
                                                      int r, int32_t *umap, int32_t *moff, int32_t *midx,
                                                      int32_t *kept) {
    extern __shared__ __align__(16) unsigned char tm_sm[];
    float *bs = (float *)tm_sm;                 // [n_a]
    int *bb = (int *)(bs + n_a);                // [n_a]
    int *mg = bb + n_a;                         // [n_a] merged flag
    int *cnt = mg + n_a;                        // [n_b] merged A rows per B row
    const int w = blockIdx.x, t = threadIdx.x;
    for (int a = t; a < n_a; a += 1024) {
        const unsigned long long *kp = keys + ((size_t)w * n_a + a) * nbt;
        unsigned long long m = 0ull;
        for (int i = 0; i < nbt; i++) m = kp[i] > m ? kp[i] : m;
        bb[a] = m ? (int)(0xffffffffu - (uint32_t)m) : 0;
        bs[a] = m ? tm_key_value(m) : -INFINITY;
    }
    __syncthreads();
    for (int a = t; a < n_a; a += 1024) {
        const float v = bs[a];
        int rk = 0;
        for (int j = 0; j < n_a; j++) rk += (bs[j] > v || (j < a && bs[j] == v)) ? 1 : 0;
        mg[a] = rk < r;
    }
    __syncthreads();
    for (int b = t; b < n_b; b += 1024) {
        int c = 0;
        for (int a = 0; a < n_a; a++) c += (mg[a] && bb[a] == b) ? 1 : 0;
        cnt[b] = c;
    }
    __syncthreads();
    int32_t *mo = moff + (size_t)w * (n_b + 1), *mi = midx + (size_t)w * n_a, *kp = kept + (size_t)w * n_a;
    int32_t *um = umap + (size_t)w * T;
    for (int b = t; b < n_b; b += 1024) {
        int o = 0;
        for (int j = 0; j < b; j++) o += cnt[j];
        mo[b] = o;
        if (b == n_b - 1) mo[n_b] = o + cnt[b];
        for (int a = 0; a < n_a; a++)
            if (mg[a] && bb[a] == b) mi[o++] = a;
        um[2 * b + 1] = b;
    }
    for (int a = t; a < n_a; a += 1024) {
        if (mg[a]) {
            um[2 * a] = bb[a];
        } else {
            int s = 0;
            for (int j = 0; j < a; j++) s += mg[j] ? 0 : 1;
            um[2 * a] = n_b + s;
            kp[s] = a;
        }
    }
}

// merged row m of window w: B row m plus its merged A rows in ascending A
// order, divided by the count when it exceeds one; or the kept A row
__global__ void __launch_bounds__(256) k_tome_merge(const float *x, int T, int d, int n_b, int Tm,
                                                    const int32_t *moff, const int32_t *midx, const int32_t *kept,
                                                    int n_a, float *xm) {
    const int m = blockIdx.x, w = blockIdx.y;
    const float *xw = x + (size_t)w * T * d;
    float4 *out = (float4 *)(xm + ((size_t)w * Tm + m) * d);
    const int n4 = d >> 2;
    if (m < n_b) {
        const int32_t *mo = moff + (size_t)w * (n_b + 1), *mi = midx + (size_t)w * n_a;
        const int i0 = mo[m], i1 = mo[m + 1];
        const float c = (float)(i1 - i0 + 1);
        for (int i = threadIdx.x; i < n4; i += 256) {
            float4 v = ((const float4 *)(xw + (size_t)(2 * m + 1) * d))[i];
            for (int j = i0; j < i1; j++) {
                const float4 u = ((const float4 *)(xw + (size_t)(2 * mi[j]) * d))[i];
                v.x = v.x + u.x;
                v.y = v.y + u.y;
                v.z = v.z + u.z;
                v.w = v.w + u.w;
            }
            if (i1 > i0) {
                v.x = v.x / c;
                v.y = v.y / c;
                v.z = v.z / c;
                v.w = v.w / c;
            }
            out[i] = v;
        }
    } else {
        const int a = kept[(size_t)w * n_a + (m - n_b)];
        for (int i = threadIdx.x; i < n4; i += 256) out[i] = ((const float4 *)(xw + (size_t)(2 * a) * d))[i];
    }
}

// out[w][p] = xm[w][umap[w][p]]
__global__ void __launch_bounds__(256) k_tome_unmerge(const float *xm, int Tm, const int32_t *umap, int T, int d,
                                                      float *out) {
    const int p = blockIdx.x, w = blockIdx.y;
    const int m = umap[(size_t)w * T + p];
    const float4 *src = (const float4 *)(xm + ((size_t)w * Tm + m) * d);
    float4 *dst = (float4 *)(out + ((size_t)w * T + p) * d);
    for (int i = threadIdx.x; i < (d >> 2); i += 256) dst[i] = src[i];
}

// cum[w][p] = step[w][cum[w][p]] for the T0 original rows of every window:
// original row -> row after the latest merge (step: [B, Tprev])
__global__ void __launch_bounds__(256) k_tome_compose(int32_t *cum, const int32_t *step, int B, int T0, int Tprev) {
    const size_t n = (size_t)B * T0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        cum[i] = step[(i / T0) * Tprev + cum[i]];
}

// zero the columns [T, Tp) of V^T rows [rows, Tp] (f16)
__global__ void __launch_bounds__(256) k_tome_vpad(uint16_t *vt, size_t rows, int T, int Tp) {
    const int np = Tp - T;
    const size_t n = rows * np;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        vt[(i / np) * Tp + T + i % np] = 0;
}

} // namespace

bool fw_tome_ok(int T, int d) { return T >= 2 && T <= 4096 && d % TM_KC == 0; }

void fw_launch_tome_vpad(hipStream_t st, uint16_t *vt, size_t rows, int T, int Tp) {
    if (Tp <= T) return;
    const size_t n = rows * (size_t)(Tp - T);
    size_t g = (n + 255) / 256;
    g = g < 4096 ? g : 4096;
    hipLaunchKernelGGL(k_tome_vpad, dim3((unsigned)g), dim3(256), 0, st, vt, rows, T, Tp);
}

size_t fw_tome_ws_bytes(int B, int T) {
    const size_t n_a = (T + 1) / 2, n_b = T / 2, nbt = (n_b + TM_TILE - 1) / TM_TILE;
    return 256 + sizeof(float) * B * T + sizeof(unsigned long long) * B * n_a * nbt +
           sizeof(int32_t) * B * ((n_b + 1) + 2 * n_a) + 4 * 256;
}

// Merge x [B, T, d] into xm [B, T - r', d] (r' = min(r, n_a, T - 1)) with the
// unmerge map umap [B, T]; ws holds fw_tome_ws_bytes(B, T).  Returns T - r'.
int fw_launch_tome_merge(hipStream_t st, const float *x, int B, int T, int d, int r, void *ws, float *xm,
                         int32_t *umap) {
    const int n_a = (T + 1) / 2, n_b = T / 2, nbt = (n_b + TM_TILE - 1) / TM_TILE, nat = (n_a + TM_TILE - 1) / TM_TILE;
    if (r > n_a) r = n_a;
    if (r > T - 1) r = T - 1;
    const int Tm = T - r;
    char *p = (char *)ws;
    auto take = [&](size_t bytes) {
        char *q = p;
        p += (bytes + 255) & ~(size_t)255;
        return (void *)q;
    };
    float *nrm = (float *)take(sizeof(float) * B * T);
    unsigned long long *keys = (unsigned long long *)take(sizeof(unsigned long long) * (size_t)B * n_a * nbt);
    int32_t *moff = (int32_t *)take(sizeof(int32_t) * (size_t)B * (n_b + 1));
    int32_t *midx = (int32_t *)take(sizeof(int32_t) * (size_t)B * n_a);
    int32_t *kept = (int32_t *)take(sizeof(int32_t) * (size_t)B * n_a);
    hipLaunchKernelGGL(k_tome_norm, dim3((B * T + 255) / 256), dim3(256), 0, st, x, B * T, d, nrm);
    hipLaunchKernelGGL(k_tome_sim, dim3(nbt, nat, B), dim3(256), 0, st, x, nrm, T, d, n_a, n_b, nbt, keys);
    const size_t shm = sizeof(float) * n_a + sizeof(int) * (2 * n_a + n_b);
    hipLaunchKernelGGL(k_tome_select, dim3(B), dim3(1024), shm, st, keys, T, n_a, n_b, nbt, r, umap, moff, midx, kept);
    hipLaunchKernelGGL(k_tome_merge, dim3(Tm, B), dim3(256), 0, st, x, T, d, n_b, Tm, moff, midx, kept, n_a, xm);
    return Tm;
}

void fw_launch_tome_unmerge(hipStream_t st, const float *xm, int B, int Tm, const int32_t *umap, int T, int d,
                            float *out) {
    hipLaunchKernelGGL(k_tome_unmerge, dim3(T, B), dim3(256), 0, st, xm, Tm, umap, T, d, out);
}

void fw_launch_tome_compose(hipStream_t st, int32_t *cum, const int32_t *step, int B, int T0, int Tprev) {
    const size_t n = (size_t)B * T0;
    size_t g = (n + 255) / 256;
    g = g < 4096 ? g : 4096;
    hipLaunchKernelGGL(k_tome_compose, dim3((unsigned)g), dim3(256), 0, st, cum, step, B, T0, Tprev);
}
