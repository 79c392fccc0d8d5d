// dec_window.hip — the window decode loop on the device: process_logits in
// full (decode.rs:702-867: suppression rules, timestamp pairing, the initial
// timestamp cap, the monotone timestamp floor, the user token budget and the
// timestamp-mass forcing rule), argmax, and the loop's own state updates
// (decode.rs:3486-3566: the sliding seek delta, the going-back-in-time bail,
// end of text, the budget and end-of-audio ends, the unclosed-window rescue),
// one block per stream and step, so the host sees finished windows only.
//
// The token of a step needs the log-softmax only through the forcing rule,
// and there the comparison ts_logprob > max_text_logprob is all but
// independent of the log-sum-exp L: both sides subtract L, so L reaches the
// difference only through roundings of values of size |l - L| (a few ulp, well
// under 1e-4) and through the timestamp terms exp(lp_i - lp_max), whose
// arguments cancel L the same way.  k_win_select therefore decides from L
// formed by a tree sum and recomputes L exactly as the reference does — one
// sequential f32 sum of the exp terms in index order — only when the margin
// is within TAU = 1e-3 of zero (or in exact mode).  The per-token log
// probabilities the window statistics need (avg_logprob, segment confidence)
// come after the loop from the stored filtered rows, with the exact L
// (k_win_plogs), and so does the no-speech probability of the prefill row.
#include "fw_dec.h"
#include "fw_kernels.h"

#define WIN_BT 256 // threads per block
#ifndef WIN_UPT
#define WIN_UPT 16 // lanes per thread: WIN_NB * WIN_BT * WIN_UPT covers the vocabulary
#endif
#define WIN_TAU 1.0e-3f

namespace {

__device__ __forceinline__ float win_san(float v) { return (v - v == 0.0f) ? v : -INFINITY; } // non-finite -> -inf

__device__ __forceinline__ float wave_fmax(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_fsum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// The step's masks (decode.rs:702-867) as ranges: text [0, txt_hi),
// timestamps [ts_lo, V), the monotone floor [beg, floor_hi), plus the control
// and language tokens and, at the first step, blank and end-of-text.
struct WinMask {
    int txt_hi, ts_lo, floor_hi;
    bool initial;
};
__device__ __forceinline__ bool win_masked(int j, const FwWinCfg &c, const WinMask &k) {
    return j < k.txt_hi || j >= k.ts_lo || (j >= c.beg && j < k.floor_hi) ||
           (k.initial && (j == c.eot || j == c.space)) || j == c.no_ts || j == c.sot || j == c.no_speech ||
           j == c.solm || j == c.translate || j == c.transcribe || j == c.sot_prev || (j > c.sot && j <= c.sot + c.n_lang);
}
// the filtered, sanitized value of lane j (non-finite and masked lanes -> -inf)
__device__ __forceinline__ float win_u(const float *lg, int j, const FwWinCfg &c, const WinMask &k) {
    return win_masked(j, c, k) ? -INFINITY : win_san(lg[j]);
}

// the forcing rule for log-sum-exp `lse` (decode.rs:845-864): returns
// ts_logprob - max_text_logprob (>0: force a timestamp); the timestamp lanes
// are formed again from the raw row; E holds the timestamp terms, bc a
// broadcast slot
__device__ float win_margin(const float *lg, const FwWinCfg &c, const WinMask &k, float lse, float mtxt, float mts,
                            float *E, float *bc) {
    const int tid = threadIdx.x, nts = c.V - c.beg;
    const float lpmax = mts - lse;
    // the lanes' raw values requested together (clamped indices, no load
    // behind a branch), then filtered
    constexpr int PT = (WIN_MAXTS + 4 + WIN_BT - 1) / WIN_BT;
    float raw[PT];
#pragma unroll
    for (int q = 0; q < PT; q++) {
        const int j = tid + q * WIN_BT;
        raw[q] = lg[c.beg + (j < nts ? j : nts - 1)];
    }
#pragma unroll
    for (int q = 0; q < PT; q++) {
        const int j = tid + q * WIN_BT;
        if (j < nts + 4) {
            float e = 0.0f;
            if (j < nts) {
                const float u = win_masked(c.beg + j, c, k) ? -INFINITY : win_san(raw[q]);
                if (u > -INFINITY) e = fw_expf((u - lse) - lpmax);
            }
            E[j] = e;
        }
    }
    __syncthreads();
    if (tid < 64) {
        const float sts = fw_seq_sum_wave(E, nts);
        if (tid == 0) bc[0] = sts;
    }
    __syncthreads();
    const float sts = bc[0];
    __syncthreads();
    const float ts_lp = sts > 0.0f ? fw_logf(sts) + lpmax : -INFINITY;
    const float max_text = mtxt - lse;
    return ts_lp - max_text;
}

template <int NW>
__device__ __forceinline__ float block_fmax(float v, float *sh) {
    v = wave_fmax(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    float r = sh[0];
#pragma unroll
    for (int w = 1; w < NW; w++) r = fmaxf(r, sh[w]);
    return r;
}

} // namespace

// One step of the window loop.  Grid (WIN_NB, streams): block b of stream s
// filters lanes [b * CH, (b + 1) * CH) of the row (masks, stored row, argmax
// keys of all lanes and of the timestamp lanes, maxima, and with timestamps
// the sum of expf(u - m_b) over its lanes against its own maximum m_b), writes
// them to its slot of `part`, and counts itself in; the block that counts last
// merges the slots in block order (log-sum-exp sum_b s_b expf(m_b - M) for the
// decision), runs the forcing rule, the exact fallback and the loop state.
// The counter is reset by that block, so every launch starts from zero.
__global__ void __launch_bounds__(WIN_BT) k_win_select(const float *__restrict__ logits, int ldl, FwWinCfg c,
                                                       FwWinStream *ws, int32_t *hist, int hist_cap, float *rows,
                                                       uint8_t *forced, float *scratch, int32_t *tok_out, int *posp,
                                                       int *ndone, FwWinPart *part, int *cnt) {
    constexpr int NW = WIN_BT / 64;
    const int b = blockIdx.x, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    __shared__ __align__(16) float E[WIN_MAXTS + 8];
    __shared__ unsigned long long kred[NW][2];
    __shared__ float fred[NW][4];
    __shared__ float bc[2];
    __shared__ int last;
    if (s == 0 && b == 0 && tid == 0) *posp = *posp + 1; // the next forward's position
    const FwWinStream st = ws[s];
    if (st.done) {
        if (b == 0 && tid == 0) tok_out[s] = c.eot; // a valid token for the forward nobody reads
        return;
    }
    const int i = st.n_dec;
    const int32_t *prev = hist + (size_t)s * hist_cap;
    WinMask mk;
    mk.initial = i == 0;
    const bool last_ts = i > 0 && prev[i - 1] >= c.beg;
    const bool penult_ts = i < 2 || prev[i - 2] >= c.beg;
    mk.txt_hi = 0;
    mk.ts_lo = c.V;
    if (!c.timestamps) mk.ts_lo = c.beg;
    if (c.timestamps && c.max_tokens > 0 && i >= c.max_tokens) mk.txt_hi = c.eot;
    if (last_ts) {
        if (penult_ts) mk.ts_lo = min(mk.ts_lo, c.beg);
        else mk.txt_hi = max(mk.txt_hi, c.eot);
    }
    if (mk.initial && c.max_initial_tid >= 0) mk.ts_lo = min(mk.ts_lo, c.beg + c.max_initial_tid + 1);
    mk.floor_hi = st.has_ts ? min(c.beg + st.seek_delta_cs / 2, c.V) : c.beg;

    const float *lg = logits + (size_t)s * ldl;
    float *row = rows + ((size_t)s * c.n_max + i) * c.ldr;
    const int CH = ((c.V + WIN_NB * WIN_BT - 1) / (WIN_NB * WIN_BT)) * WIN_BT; // lanes per block
    const int j0 = b * CH, j1 = min(c.V, j0 + CH);
    unsigned long long ka = 0ull, kt = 0ull;
    float mall = -INFINITY, mtxt = -INFINITY, mts = -INFINITY;
    float uv[WIN_UPT];
    // every lane's value requested at once (clamped indices: no load behind a
    // branch, so no load waits for the one before it)
#pragma unroll
    for (int q = 0; q < WIN_UPT; q++) {
        const int j = j0 + q * WIN_BT + tid;
        uv[q] = lg[j < j1 ? j : j1 - 1];
    }
#pragma unroll
    for (int q = 0; q < WIN_UPT; q++) {
        const int j = j0 + q * WIN_BT + tid;
        if (j < j1) {
            float v = uv[q];
            uv[q] = -INFINITY;
            if (win_masked(j, c, mk)) v = -INFINITY;
            row[j] = v;
            const unsigned long long k = am_key(v, j);
            ka = k > ka ? k : ka;
            const float u = win_san(v);
            uv[q] = u;
            mall = fmaxf(mall, u);
            if (j < c.beg) {
                mtxt = fmaxf(mtxt, u);
            } else {
                kt = k > kt ? k : kt;
                mts = fmaxf(mts, u);
            }
        } else {
            uv[q] = -INFINITY;
        }
    }
    ka = wave_max_u64(ka);
    kt = wave_max_u64(kt);
    mall = wave_fmax(mall);
    mtxt = wave_fmax(mtxt);
    mts = wave_fmax(mts);
    if (lane == 0) {
        kred[wave][0] = ka;
        kred[wave][1] = kt;
        fred[wave][0] = mall;
        fred[wave][1] = mtxt;
        fred[wave][2] = mts;
    }
    __syncthreads();
    ka = kt = 0ull;
    mall = mtxt = mts = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        ka = kred[w][0] > ka ? kred[w][0] : ka;
        kt = kred[w][1] > kt ? kred[w][1] : kt;
        mall = fmaxf(mall, fred[w][0]);
        mtxt = fmaxf(mtxt, fred[w][1]);
        mts = fmaxf(mts, fred[w][2]);
    }
    // the block's exp sum against its own maximum (the decision's estimate)
    float sb = 0.0f;
    if (c.timestamps && mall > -INFINITY) {
#pragma unroll
        for (int q = 0; q < WIN_UPT; q++)
            if (uv[q] > -INFINITY) sb += fw_expf(uv[q] - mall);
        sb = wave_fsum(sb);
        __syncthreads();
        if (lane == 0) fred[wave][3] = sb;
        __syncthreads();
        sb = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; w++) sb += fred[w][3];
    }
    if (tid == 0) {
        FwWinPart o;
        o.ka = ka;
        o.kt = kt;
        o.mall = mall;
        o.mtxt = mtxt;
        o.mts = mts;
        o.sb = sb;
        part[(size_t)s * WIN_NB + b] = o;
        __threadfence(); // the slot is visible device-wide before the count
        last = atomicAdd(cnt + s, 1) == WIN_NB - 1;
    }
    __syncthreads();
    if (!last) return;
    __threadfence(); // every other block's slot is visible to this block
    // lane q of every wave holds slot q; the maxima by lane exchanges, the
    // sum in slot order
    FwWinPart pq = part[(size_t)s * WIN_NB + (lane < WIN_NB ? lane : 0)];
    if (lane >= WIN_NB) {
        pq.ka = pq.kt = 0ull;
        pq.mall = pq.mtxt = pq.mts = -INFINITY;
        pq.sb = 0.0f;
    }
    ka = wave_max_u64(pq.ka);
    kt = wave_max_u64(pq.kt);
    mall = wave_fmax(pq.mall);
    mtxt = wave_fmax(pq.mtxt);
    mts = wave_fmax(pq.mts);
    float sa = 0.0f;
    {
        const float t = pq.mall > -INFINITY ? pq.sb * fw_expf(pq.mall - mall) : 0.0f;
#pragma unroll
        for (int q = 0; q < WIN_NB; q++) sa += __shfl(t, q, 64);
    }

    // the forcing rule; with every timestamp lane masked it cannot fire
    // (ts_logprob stays -inf), so no-timestamps mode skips it
    bool force = false, used_exact = false;
    if (c.timestamps && mts > -INFINITY) {
        float mg = win_margin(lg, c, mk, fw_logf(sa) + mall, mtxt, mts, E, bc);
        if (c.exact || fabsf(mg) <= WIN_TAU) {
            // the reference's own log-sum-exp: expf(l - max) over the finite
            // lanes summed sequentially in index order (masked lanes add +0)
            float *sc = scratch + (size_t)s * c.ldr;
            for (int j = tid; j < c.V; j += WIN_BT) {
                const float u = win_u(lg, j, c, mk);
                sc[j] = u > -INFINITY ? fw_expf(u - mall) : 0.0f;
            }
            __threadfence_block();
            __syncthreads();
            if (tid == 0) {
                float sum = 0.0f;
                int j = 0;
                for (; j + 8 <= c.V; j += 8) {
                    const float4 a = *(const float4 *)(sc + j), e = *(const float4 *)(sc + j + 4);
                    sum = sum + a.x;
                    sum = sum + a.y;
                    sum = sum + a.z;
                    sum = sum + a.w;
                    sum = sum + e.x;
                    sum = sum + e.y;
                    sum = sum + e.z;
                    sum = sum + e.w;
                }
                for (; j < c.V; j++) sum = sum + sc[j];
                bc[1] = fw_logf(sum) + mall;
            }
            __syncthreads();
            mg = win_margin(lg, c, mk, bc[1], mtxt, mts, E, bc);
            used_exact = true;
        }
        force = mg > 0.0f;
    }

    if (tid == 0) {
        cnt[s] = 0; // every block of this stream has counted: ready for the next launch
        const unsigned long long k = force ? kt : ka;
        const int tok = k ? (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull)) : 0;
        hist[(size_t)s * hist_cap + i] = tok;
        forced[(size_t)s * c.n_max + i] = force ? 1 : 0;
        int done = 0, has_ts = st.has_ts, delta = st.seek_delta_cs, rl = st.result_len;
        if (tok > c.beg) {
            const int nd = 2 * (tok - c.beg);
            if (has_ts && delta > nd && rl < i) {
                done = 1; // going back in time: bail out of the window
            } else {
                delta = nd;
                rl = i + 1;
                has_ts = 1;
            }
        }
        if (!done) {
            const bool budget = c.max_tokens > 0 && i >= c.max_tokens;
            const bool covers = (long long)st.seek_cs + delta + 10 >= (long long)st.seek_end_cs;
            if (tok == c.eot || budget || (has_ts && covers)) {
                if (rl == 0 && c.timestamps && covers && (st.seek_cs == 0 || !st.has_prior)) rl = i + 1;
                if (!c.timestamps) {
                    rl = i + 1;
                    delta = 3000;
                }
                done = 1;
            } else if (i + 1 >= c.n_max) {
                done = 1;
            }
        }
        FwWinStream o = st;
        o.n_dec = i + 1;
        o.has_ts = has_ts;
        o.seek_delta_cs = delta;
        o.result_len = rl;
        o.done = done;
        o.n_exact = st.n_exact + (used_exact ? 1 : 0);
        ws[s] = o;
        tok_out[s] = tok;
        if (done) atomicAdd(ndone, 1);
    }
}

// Log-probability of every sampled token (row r = s * (n_max + 1) + i, i <
// n_dec) and of the no-speech token on the raw prefill row (i == n_max):
// compute_logprobs (decode.rs:1666-1701) of the row — non-finite lanes as
// -inf, max, expf(l - max) summed sequentially in index order, logf + max —
// at the chosen lane; -inf for a text token of a forced step (the forcing
// rule set those log-probabilities to -inf).
__global__ void __launch_bounds__(256) k_win_plogs(const float *__restrict__ rows, const float *__restrict__ nsrow,
                                                   FwWinCfg c, const FwWinStream *ws, const int32_t *hist,
                                                   int hist_cap, const uint8_t *forced, float *plogs, float *nslp) {
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int s = r / (c.n_max + 1), i = r % (c.n_max + 1);
    const bool ns = i == c.n_max;
    if (!ns && i >= ws[s].n_dec) return;
    const float *row = ns ? nsrow + (size_t)s * c.ldr : rows + ((size_t)s * c.n_max + i) * c.ldr;
    const int tok = ns ? c.no_speech : hist[(size_t)s * hist_cap + i];
    __shared__ __align__(16) float tile[1024];
    __shared__ float red[4];
    float m = -INFINITY;
    for (int j = tid; j < c.V; j += 256) m = fmaxf(m, win_san(row[j]));
    m = wave_fmax(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.0f; // thread 0's running sum
    for (int j0 = 0; j0 < c.V; j0 += 1024) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int j = j0 + q * 256 + tid;
            float e = 0.0f;
            if (j < c.V) {
                const float u = win_san(row[j]);
                if (u > -INFINITY) e = fw_expf(u - m);
            }
            tile[q * 256 + tid] = e;
        }
        __syncthreads();
        if (tid == 0) {
            const int n = c.V - j0 < 1024 ? c.V - j0 : 1024;
            int k = 0;
            for (; k + 4 <= n; k += 4) {
                const float4 v = *(const float4 *)(tile + k);
                sum = sum + v.x;
                sum = sum + v.y;
                sum = sum + v.z;
                sum = sum + v.w;
            }
            for (; k < n; k++) sum = sum + tile[k];
        }
    }
    if (tid == 0) {
        const float lse = fw_logf(sum) + m;
        const float u = (tok >= 0 && tok < c.V) ? win_san(row[tok]) : -INFINITY;
        float lp = u > -INFINITY ? u - lse : -INFINITY;
        if (!ns && forced[(size_t)s * c.n_max + i] && tok < c.beg) lp = -INFINITY;
        if (ns) nslp[s] = lp;
        else plogs[(size_t)s * c.n_max + i] = lp;
    }
}

bool fw_win_select_ok(int V) { return V > 0 && V <= WIN_NB * WIN_BT * WIN_UPT; }

void fw_launch_win_select(hipStream_t st, const float *logits, int ldl, const FwWinCfg &c, FwWinStream *ws,
                          int32_t *hist, int hist_cap, float *rows, uint8_t *forced, float *scratch, int32_t *tok,
                          int *posp, int *ndone, FwWinPart *part, int *cnt, int ns) {
    hipLaunchKernelGGL(k_win_select, dim3(WIN_NB, ns), dim3(WIN_BT), 0, st, logits, ldl, c, ws, hist, hist_cap, rows,
                       forced, scratch, tok, posp, ndone, part, cnt);
}

void fw_launch_win_plogs(hipStream_t st, const float *rows, const float *nsrow, const FwWinCfg &c,
                         const FwWinStream *ws, const int32_t *hist, int hist_cap, const uint8_t *forced,
                         float *plogs, float *nslp, int ns) {
    hipLaunchKernelGGL(k_win_plogs, dim3(ns * (c.n_max + 1)), dim3(256), 0, st, rows, nsrow, c, ws, hist, hist_cap,
                       forced, plogs, nslp);
}
