// ggml.hip — whisper.cpp ggml model files on the GPU engine.
//
//  - The directory scan of GgmlModel::load (ggml.rs:903-1136, the streamed
//    variant 1160-1220): magic, the eleven hparams, the mel filterbank, the
//    byte-level vocab and the tensor directory, read through a bounds-checked
//    cursor over pread (the payloads stay in the file until a tensor is asked
//    for) or over caller memory (GgmlModel::from_bytes, ggml.rs:953).  Errors
//    carry the reference's messages and classes.
//  - GPU dequantization of every element type the reference decodes
//    (tensor_f32, ggml.rs:1478-1632: f32, f16, q4_0, q4_1, q5_0, q5_1, q8_0,
//    q2_k, q3_k, q4_k, q5_k, q6_k).  A workgroup stages a tile of whole
//    blocks through LDS with dword loads and writes 1024 f32 outputs with
//    fully coalesced stores; each output is decoded from its block position.
//    The arithmetic is the reference's, one rounding per operation.
//  - The encoder / decoder loads of EncoderWeights::from_ggml (encoder.rs:764)
//    and DecoderWeights::from_ggml (decoder.rs:752): names, shapes and error
//    messages of the reference, feeding fwhip_encoder_load /
//    fwhip_decoder_load.  The GPU arms compute with binary16 weights, so a
//    linear stored in another type is accepted by the encoder only when every
//    value is a binary16 value (then the reference computes on the same
//    numbers); the decoder's arms are the reference's f16-stored arms
//    (decoder.rs:606-609, 675-681), so the decoder needs f16-stored linears.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cinttypes>
#include <cstdio>

#include "fw_internal.h"

#define GG_HIP(expr)                                                                          \
    do {                                                                                      \
        hipError_t _e = (expr);                                                               \
        if (_e != hipSuccess)                                                                 \
            return fw_fail(FWHIP_ERR_GENERIC, std::string(#expr ": ") + hipGetErrorString(_e)); \
    } while (0)

namespace {

constexpr uint32_t GGML_MAGIC = 0x67676d6cu;
constexpr int GGML_MAX_DIMS = 4;

struct TypeInfo {
    int qk, bb;
    const char *name;
};

// ttype -> block geometry (ggml.rs:66-111, 386-474); qk == 0 marks an
// unsupported code
static TypeInfo type_info(int t) {
    switch (t) {
    case 0: return {1, 4, "f32"};
    case 1: return {1, 2, "f16"};
    case 2: return {32, 18, "q4_0"};
    case 3: return {32, 20, "q4_1"};
    case 6: return {32, 22, "q5_0"};
    case 7: return {32, 24, "q5_1"};
    case 8: return {32, 34, "q8_0"};
    case 10: return {256, 84, "q2_k"};
    case 11: return {256, 110, "q3_k"};
    case 12: return {256, 144, "q4_k"};
    case 13: return {256, 176, "q5_k"};
    case 14: return {256, 210, "q6_k"};
    default: return {0, 0, ""};
    }
}

struct GgErr {
    fwhip_status code;
    std::string msg;
};

[[noreturn]] static void gg_throw(fwhip_status code, const std::string &msg) { throw GgErr{code, msg}; }

static std::string fmt_shape(const std::vector<uint64_t> &s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); i++) {
        if (i) r += ", ";
        r += std::to_string(s[i]);
    }
    return r + "]";
}

// ggml_byte_len (ggml.rs:386-474)
static uint64_t byte_len(int t, uint64_t n, const std::string &name) {
    TypeInfo ti = type_info(t);
    if (ti.qk > 1 && n % (uint64_t)ti.qk)
        gg_throw(FWHIP_ERR_INVALID, "tensor '" + name + "' " + ti.name + " element count " + std::to_string(n) +
                                        " is not a multiple of " + std::to_string(ti.qk));
    uint64_t v;
    if (__builtin_mul_overflow(n / (uint64_t)ti.qk, (uint64_t)ti.bb, &v))
        gg_throw(FWHIP_ERR_INVALID, "tensor '" + name + "' byte length overflow");
    return v;
}

} // namespace

struct GgmlEntry {
    std::vector<uint64_t> shape; // logical (row-major) order: ggml's ne[] reversed
    int32_t dtype;
    uint64_t off, len;
};

struct fwhip_ggml {
    int fd = -1;
    const uint8_t *mem = nullptr; // the from-bytes source (a private copy)
    std::vector<uint8_t> mem_copy;
    uint64_t size = 0;
    int32_t hp[11] = {};
    int32_t n_mel = 0, n_fft = 0;
    std::vector<float> filters;
    std::vector<std::string> vocab;
    std::map<std::string, GgmlEntry> tensors; // name order (tensor_names is sorted)
    std::vector<const std::string *> by_index;

    ~fwhip_ggml() {
        if (fd >= 0) close(fd);
    }

    // positioned read of [off, off + n) into dst (the file or the memory copy)
    void pread_exact(void *dst, uint64_t n, uint64_t off, const std::string &what) const {
        if (mem) {
            memcpy(dst, mem + off, n);
            return;
        }
        uint8_t *p = (uint8_t *)dst;
        while (n) {
            size_t chunk = n > (1u << 30) ? (1u << 30) : (size_t)n;
            ssize_t r = pread(fd, p, chunk, (off_t)off);
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0)
                gg_throw(FWHIP_ERR_INVALID,
                         what + " pread failed: " + (r < 0 ? std::string(strerror(errno)) : "unexpected end of file"));
            p += r;
            off += (uint64_t)r;
            n -= (uint64_t)r;
        }
    }
};

namespace {

// Cursor / StreamCursor (ggml.rs:1947-2098): little-endian reads bounded by the
// source length, buffered 64 KiB at a time over pread; payloads are skipped.
struct Cursor {
    const fwhip_ggml &g;
    uint64_t pos = 0;
    std::vector<uint8_t> buf;
    uint64_t buf_off = 0, buf_len = 0;

    explicit Cursor(const fwhip_ggml &src) : g(src) {}

    bool at_end() const { return pos >= g.size; }
    uint64_t remaining() const { return g.size > pos ? g.size - pos : 0; }

    void need(uint64_t n) const {
        uint64_t end;
        if (__builtin_add_overflow(pos, n, &end)) gg_throw(FWHIP_ERR_INVALID, "read length overflow");
        if (end > g.size)
            gg_throw(FWHIP_ERR_INVALID, "unexpected end of file: needed " + std::to_string(n) + " byte(s) at offset " +
                                            std::to_string(pos) + ", have " + std::to_string(g.size));
    }

    void read(void *dst, uint64_t n) {
        need(n);
        if (g.mem) {
            memcpy(dst, g.mem + pos, n);
            pos += n;
            return;
        }
        uint8_t *p = (uint8_t *)dst;
        while (n) {
            if (pos < buf_off || pos >= buf_off + buf_len) {
                uint64_t len = g.size - pos < (64u << 10) ? g.size - pos : (64u << 10);
                buf.resize(len);
                g.pread_exact(buf.data(), len, pos, "ggml directory");
                buf_off = pos;
                buf_len = len;
            }
            uint64_t k = buf_off + buf_len - pos;
            if (k > n) k = n;
            memcpy(p, buf.data() + (pos - buf_off), k);
            p += k;
            pos += k;
            n -= k;
        }
    }

    void skip(uint64_t n) {
        need(n);
        pos += n;
    }
    uint32_t u32() {
        uint8_t b[4];
        read(b, 4);
        return (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
    }
    int32_t i32() { return (int32_t)u32(); }
};

static uint64_t usize_from(int32_t v, const char *what) {
    if (v < 0) gg_throw(FWHIP_ERR_INVALID, std::string(what) + " is negative (" + std::to_string(v) + ")");
    return (uint64_t)v;
}

// GgmlModel::parse / scan_streamed_inner (ggml.rs:982-1136)
static void scan(fwhip_ggml &g) {
    Cursor cur(g);
    uint32_t magic = cur.u32();
    if (magic != GGML_MAGIC) {
        char m[96];
        snprintf(m, sizeof m, "bad ggml magic: got %#010x, expected %#010x", magic, GGML_MAGIC);
        gg_throw(FWHIP_ERR_INVALID, m);
    }
    for (int i = 0; i < 11; i++) g.hp[i] = cur.i32();
    int32_t base = ((g.hp[10] % 1000) + 1000) % 1000; // rem_euclid(GGML_QNT_VERSION_FACTOR)
    static const int ok_base[] = {0, 1, 2, 3, 7, 8, 9, 10, 11, 12, 13, 14};
    bool ok = false;
    for (int b : ok_base) ok = ok || b == base;
    if (!ok)
        gg_throw(FWHIP_ERR_UNSUPPORTED,
                 "quantized ggml ftype " + std::to_string(g.hp[10]) + " (base " + std::to_string(base) +
                     ") is not supported (only base 0=f32, 1=f16, 2=q4_0, 3=q4_1, 7=q8_0, 8=q5_0, 9=q5_1, "
                     "10=q2_k, 11=q3_k, 12=q4_k, 13=q5_k, 14=q6_k)");
    int32_t nm = cur.i32(), nf = cur.i32();
    uint64_t n_mel = usize_from(nm, "filters.n_mel"), n_fft = usize_from(nf, "filters.n_fft");
    uint64_t n_filter = n_mel * n_fft; // both < 2^31: no overflow
    if (cur.remaining() / 4 < n_filter) {
        // the reference reads one f32 at a time and stops at the first short read
        cur.pos += (cur.remaining() / 4) * 4;
        cur.need(4);
    }
    g.n_mel = nm;
    g.n_fft = nf;
    g.filters.resize(n_filter);
    cur.read(g.filters.data(), 4 * n_filter);
    uint64_t n_vocab = usize_from(cur.i32(), "file vocab count");
    g.vocab.reserve(n_vocab < cur.remaining() / 4 ? n_vocab : cur.remaining() / 4);
    for (uint64_t i = 0; i < n_vocab; i++) {
        uint32_t len = cur.u32();
        cur.need(len);
        std::string tok(len, '\0');
        cur.read(tok.data(), len);
        g.vocab.push_back(std::move(tok));
    }
    bool nul_name = false; // a name with a NUL byte: valid UTF-8, but not a C string
    while (!cur.at_end()) {
        int32_t nd = cur.i32(), nl = cur.i32(), ttype = cur.i32();
        uint64_t n_dims = usize_from(nd, "tensor n_dims");
        if (n_dims == 0 || n_dims > (uint64_t)GGML_MAX_DIMS)
            gg_throw(FWHIP_ERR_INVALID,
                     "tensor n_dims " + std::to_string(n_dims) + " out of range 1..=" + std::to_string(GGML_MAX_DIMS));
        uint64_t name_len = usize_from(nl, "tensor name length");
        if (type_info(ttype).qk == 0)
            gg_throw(FWHIP_ERR_UNSUPPORTED, "tensor element type " + std::to_string(ttype) +
                                                " is not supported (only 0=f32, 1=f16, 2=q4_0, 3=q4_1, 6=q5_0, "
                                                "7=q5_1, 8=q8_0, 10=q2_k, 11=q3_k, 12=q4_k, 13=q5_k, 14=q6_k)");
        std::vector<uint64_t> ne(n_dims);
        for (auto &d : ne) d = usize_from(cur.i32(), "tensor dimension");
        cur.need(name_len);
        std::string name(name_len, '\0');
        cur.read(name.data(), name_len);
        // String::from_utf8: reject malformed UTF-8
        for (size_t i = 0; i < name.size();) {
            unsigned char c = (unsigned char)name[i];
            size_t k = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
            bool good = k && i + k <= name.size() && !(k == 2 && c < 0xc2) && !(k == 4 && c > 0xf4);
            for (size_t j = 1; good && j < k; j++) good = ((unsigned char)name[i + j] >> 6) == 2;
            if (good && k == 3) {
                unsigned c1 = (unsigned char)name[i + 1];
                good = !(c == 0xe0 && c1 < 0xa0) && !(c == 0xed && c1 >= 0xa0);
            }
            if (good && k == 4) {
                unsigned c1 = (unsigned char)name[i + 1];
                good = !(c == 0xf0 && c1 < 0x90) && !(c == 0xf4 && c1 >= 0x90);
            }
            if (!good) gg_throw(FWHIP_ERR_INVALID, "tensor name is not valid UTF-8");
            i += k;
        }
        nul_name = nul_name || name.find('\0') != std::string::npos;
        std::vector<uint64_t> shape(ne.rbegin(), ne.rend());
        uint64_t n = 1;
        for (uint64_t d : shape)
            if (__builtin_mul_overflow(n, d, &n)) gg_throw(FWHIP_ERR_INVALID, "tensor '" + name + "' element count overflow");
        uint64_t len = byte_len(ttype, n, name);
        uint64_t off = cur.pos;
        cur.skip(len);
        g.tensors[name] = GgmlEntry{shape, ttype, off, len};
    }
    // the reference accepts such a name; the C ABI passes names as C strings,
    // so a file the reference would load is refused here rather than read
    // with truncated names (the caller keeps its CPU route)
    if (nul_name)
        gg_throw(FWHIP_ERR_UNSUPPORTED, "cpu:ggml-nul-in-tensor-name: a tensor name holds a NUL byte, which the "
                                        "C ABI's string names cannot carry");
    for (auto &kv : g.tensors) g.by_index.push_back(&kv.first);
}

static const GgmlEntry &entry_of(const fwhip_ggml *g, const char *name, const char *unknown_fmt) {
    auto it = g->tensors.find(name);
    if (it == g->tensors.end()) gg_throw(FWHIP_ERR_INVALID, std::string(unknown_fmt) + name + "'");
    return it->second;
}

static uint64_t n_elements(const GgmlEntry &e) {
    uint64_t n = 1;
    for (uint64_t d : e.shape) n *= d;
    return n;
}

} // namespace

// ---------------------------------------------------------------------------
// device dequantization

namespace {

constexpr int DQ_TILE = 1024; // outputs per workgroup tile (4 per thread)

__device__ __forceinline__ float dq_h(const uint8_t *b, int off) {
    uint16_t h = (uint16_t)b[off] | ((uint16_t)b[off + 1] << 8);
    return (float)__builtin_bit_cast(_Float16, h);
}

// output i (0 <= i < QK) of the block at b, in the reference's arithmetic
template <int T>
__device__ __forceinline__ float dq_elem(const uint8_t *b, int i) {
    if constexpr (T == 0) {
        uint32_t u = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
        return __uint_as_float(u);
    } else if constexpr (T == 1) {
        return dq_h(b, 0);
    } else if constexpr (T == 8) { // q8_0: q * d
        return (float)(int8_t)b[2 + i] * dq_h(b, 0);
    } else if constexpr (T == 2) { // q4_0: (nibble - 8) * d
        int nib = (b[2 + (i & 15)] >> ((i >> 4) * 4)) & 15;
        return (float)(nib - 8) * dq_h(b, 0);
    } else if constexpr (T == 3) { // q4_1: nibble * d + m
        int nib = (b[4 + (i & 15)] >> ((i >> 4) * 4)) & 15;
        return (float)nib * dq_h(b, 0) + dq_h(b, 2);
    } else if constexpr (T == 6 || T == 7) { // q5_0 / q5_1: bit i of qh is bit 4 of element i
        constexpr int QH = T == 6 ? 2 : 4;
        int nib = (b[QH + 4 + (i & 15)] >> ((i >> 4) * 4)) & 15;
        int hb = (b[QH + (i >> 3)] >> (i & 7)) & 1;
        int x = nib | (hb << 4);
        if constexpr (T == 6) return (float)(x - 16) * dq_h(b, 0);
        else return (float)x * dq_h(b, 0) + dq_h(b, 2);
    } else if constexpr (T == 10) { // q2_k
        int half = i >> 7, j = (i >> 5) & 3, t = i & 31;
        int sc = b[half * 8 + 2 * j + (t >> 4)];
        int q = (b[16 + half * 32 + t] >> (2 * j)) & 3;
        float dl = dq_h(b, 80) * (float)(sc & 15), ml = dq_h(b, 82) * (float)(sc >> 4);
        return dl * (float)q - ml;
    } else if constexpr (T == 11) { // q3_k
        int half = i >> 7, j = (i >> 5) & 3, t = i & 31;
        int k = half * 8 + 2 * j + (t >> 4);
        int lo = (b[96 + (k & 7)] >> ((k >> 3) * 4)) & 15;
        int hi = (b[104 + (k & 3)] >> ((k >> 2) * 2)) & 3;
        float dl = (float)((lo | (hi << 4)) - 32) * dq_h(b, 108);
        int q = (b[32 + half * 32 + t] >> (2 * j)) & 3;
        int high = (b[t] >> (half * 4 + j)) & 1;
        return dl * (float)(q - (high ? 0 : 4));
    } else if constexpr (T == 12 || T == 13) { // q4_k / q5_k: get_scale_min_k4
        int g = i >> 6, h = (i >> 5) & 1, t = i & 31, k = 2 * g + h;
        const uint8_t *sc = b + 4;
        int s, m;
        if (k < 4) {
            s = sc[k] & 63;
            m = sc[k + 4] & 63;
        } else {
            s = (sc[k + 4] & 15) | ((sc[k - 4] >> 6) << 4);
            m = (sc[k + 4] >> 4) | ((sc[k] >> 6) << 4);
        }
        int q;
        if constexpr (T == 12) q = (b[16 + 32 * g + t] >> (4 * h)) & 15;
        else q = ((b[48 + 32 * g + t] >> (4 * h)) & 15) + (((b[16 + t] >> k) & 1) << 4);
        float dl = dq_h(b, 0) * (float)s, ml = dq_h(b, 2) * (float)m;
        return dl * (float)q - ml;
    } else { // q6_k
        int c = i >> 7, k = (i >> 5) & 3, t = i & 31;
        int lo = (b[c * 64 + t + 32 * (k & 1)] >> (4 * (k >> 1))) & 15;
        int hi = (b[128 + c * 32 + t] >> (2 * k)) & 3;
        int sc = (int8_t)b[192 + c * 8 + (t >> 4) + 2 * k];
        return (dq_h(b, 208) * (float)sc) * (float)((lo | (hi << 4)) - 32);
    }
}

template <int T, int QK, int BB>
__global__ void __launch_bounds__(256) k_dequant(const uint8_t *__restrict__ raw, uint64_t raw_bytes,
                                                  float *__restrict__ out, int64_t n) {
    constexpr int TB = DQ_TILE / QK * BB; // raw bytes of one tile (a multiple of 4)
    static_assert(TB % 4 == 0, "tile bytes");
    __shared__ uint32_t lds[TB / 4];
    const uint8_t *lb = (const uint8_t *)lds;
    const int64_t n_tiles = (n + DQ_TILE - 1) / DQ_TILE;
    for (int64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const uint64_t rb = (uint64_t)tile * TB;
        for (int w = threadIdx.x; w < TB / 4; w += 256) {
            uint64_t o = rb + 4u * (uint64_t)w;
            uint32_t v = 0;
            if (o + 4 <= raw_bytes) {
                v = *(const uint32_t *)(raw + o); // raw is 4-byte aligned (checked on the host)
            } else {
                for (int k = 0; k < 4; k++)
                    if (o + k < raw_bytes) v |= (uint32_t)raw[o + k] << (8 * k);
            }
            lds[w] = v;
        }
        __syncthreads();
        const int64_t e0 = tile * DQ_TILE;
#pragma unroll
        for (int r = 0; r < DQ_TILE / 256; r++) {
            int le = r * 256 + threadIdx.x; // consecutive lanes write consecutive floats
            if (e0 + le < n) out[e0 + le] = dq_elem<T>(lb + (le / QK) * BB, le % QK);
        }
        __syncthreads();
    }
}

template <int T>
static void launch_dq(hipStream_t st, int n_cu, const void *raw, uint64_t raw_bytes, float *out, int64_t n) {
    constexpr int QK = T == 0 || T == 1 ? 1 : (T <= 8 ? 32 : 256);
    constexpr int BB = T == 0 ? 4 : T == 1 ? 2 : T == 2 ? 18 : T == 3 ? 20 : T == 6 ? 22 : T == 7 ? 24 : T == 8 ? 34
                       : T == 10 ? 84 : T == 11 ? 110 : T == 12 ? 144 : T == 13 ? 176 : 210;
    int64_t tiles = (n + DQ_TILE - 1) / DQ_TILE;
    int64_t cap = (int64_t)n_cu * 8;
    int grid = (int)(tiles < cap ? tiles : cap);
    if (grid > 0)
        hipLaunchKernelGGL((k_dequant<T, QK, BB>), dim3(grid), dim3(256), 0, st, (const uint8_t *)raw, raw_bytes,
                           out, n);
}

// f32 -> binary16 bits (round to nearest even); *bad |= 1 where the value does
// not come back unchanged
__global__ void k_f16_exact(const float *__restrict__ x, uint16_t *__restrict__ h, int64_t n, int *bad) {
    int miss = 0;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        float v = x[i];
        _Float16 y = (_Float16)v;
        h[i] = __builtin_bit_cast(uint16_t, y);
        miss |= __float_as_uint((float)y) != __float_as_uint(v);
    }
    if (miss) atomicOr(bad, 1);
}

} // namespace

static fwhip_status dequant_launch(fwhip_ctx *c, int32_t t, const void *raw, uint64_t raw_bytes, float *out,
                                   int64_t n) {
    hipStream_t st = c->stream;
    if (!type_info(t).qk)
        return fw_fail(FWHIP_ERR_UNSUPPORTED, "tensor element type " + std::to_string(t) + " is not supported");
    // work units of the timing class: HBM bytes of the decode (payload + f32 out)
    fw_event_pair ev;
    fw_timed_begin(c, FWHIP_K_DEQUANT, (double)raw_bytes + 4.0 * (double)n, &ev);
    switch (t) {
    case 0: launch_dq<0>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 1: launch_dq<1>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 2: launch_dq<2>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 3: launch_dq<3>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 6: launch_dq<6>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 7: launch_dq<7>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 8: launch_dq<8>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 10: launch_dq<10>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 11: launch_dq<11>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 12: launch_dq<12>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 13: launch_dq<13>(st, c->n_cu, raw, raw_bytes, out, n); break;
    case 14: launch_dq<14>(st, c->n_cu, raw, raw_bytes, out, n); break;
    default: break;
    }
    fw_timed_end(c, &ev);
    GG_HIP(hipGetLastError());
    return FWHIP_OK;
}

template <class F>
static fwhip_status gg_guard(F &&f) {
    try {
        return f();
    } catch (const GgErr &e) {
        return fw_fail(e.code, e.msg);
    } catch (const std::bad_alloc &) {
        return fw_fail(FWHIP_ERR_GENERIC, "ggml: host allocation failed");
    }
}

// ---------------------------------------------------------------------------
// C ABI: file

extern "C" fwhip_status fwhip_ggml_open(const char *path, fwhip_ggml **out) {
    if (!path || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_open: NULL argument");
    *out = nullptr;
    int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fw_fail(FWHIP_ERR_GENERIC, std::string("io: ") + path + ": " + strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        int e = errno;
        close(fd);
        return fw_fail(FWHIP_ERR_GENERIC, std::string("io: ") + path + ": " + strerror(e));
    }
    fwhip_ggml *g = new fwhip_ggml();
    g->fd = fd;
    g->size = (uint64_t)sb.st_size;
    fwhip_status r = gg_guard([&] {
        scan(*g);
        return FWHIP_OK;
    });
    if (r != FWHIP_OK) {
        delete g;
        return r;
    }
    *out = g;
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_ggml_open_bytes(const void *data, uint64_t len, fwhip_ggml **out) {
    if ((!data && len) || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_open_bytes: NULL argument");
    *out = nullptr;
    fwhip_ggml *g = new fwhip_ggml();
    fwhip_status r = gg_guard([&] {
        g->mem_copy.assign((const uint8_t *)data, (const uint8_t *)data + len);
        g->mem = g->mem_copy.data();
        g->size = len;
        if (!g->mem) g->mem = (const uint8_t *)"";
        scan(*g);
        return FWHIP_OK;
    });
    if (r != FWHIP_OK) {
        delete g;
        return r;
    }
    *out = g;
    return FWHIP_OK;
}

extern "C" void fwhip_ggml_close(fwhip_ggml *g) { delete g; }

extern "C" fwhip_status fwhip_ggml_header(const fwhip_ggml *g, int32_t *hparams11) {
    if (!g || !hparams11) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_header: NULL argument");
    memcpy(hparams11, g->hp, sizeof g->hp);
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_ggml_filters(const fwhip_ggml *g, int32_t *n_mel, int32_t *n_fft_bins,
                                           const float **data) {
    if (!g || !n_mel || !n_fft_bins || !data) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_filters: NULL argument");
    *n_mel = g->n_mel;
    *n_fft_bins = g->n_fft;
    *data = g->filters.data();
    return FWHIP_OK;
}

extern "C" int32_t fwhip_ggml_vocab_count(const fwhip_ggml *g) { return g ? (int32_t)g->vocab.size() : -1; }

extern "C" fwhip_status fwhip_ggml_vocab_token(const fwhip_ggml *g, int32_t id, const uint8_t **bytes,
                                               uint32_t *len) {
    if (!g || !bytes || !len) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_vocab_token: NULL argument");
    if (id < 0 || (size_t)id >= g->vocab.size())
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_vocab_token: id " + std::to_string(id) + " out of range");
    *bytes = (const uint8_t *)g->vocab[id].data();
    *len = (uint32_t)g->vocab[id].size();
    return FWHIP_OK;
}

extern "C" int32_t fwhip_ggml_tensor_count(const fwhip_ggml *g) { return g ? (int32_t)g->by_index.size() : -1; }

extern "C" const char *fwhip_ggml_tensor_name(const fwhip_ggml *g, int32_t i) {
    if (!g || i < 0 || (size_t)i >= g->by_index.size()) return nullptr;
    return g->by_index[i]->c_str();
}

extern "C" fwhip_status fwhip_ggml_tensor_info(const fwhip_ggml *g, const char *name, int32_t *dtype, int32_t *n_dims,
                                               int64_t *shape4, uint64_t *byte_len_out) {
    if (!g || !name || !dtype || !n_dims || !shape4 || !byte_len_out)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_tensor_info: NULL argument");
    return gg_guard([&] {
        const GgmlEntry &e = entry_of(g, name, "unknown tensor '");
        *dtype = e.dtype;
        *n_dims = (int32_t)e.shape.size();
        for (int i = 0; i < 4; i++) shape4[i] = i < (int)e.shape.size() ? (int64_t)e.shape[i] : 1;
        *byte_len_out = e.len;
        return FWHIP_OK;
    });
}

extern "C" fwhip_status fwhip_ggml_tensor_raw(const fwhip_ggml *g, const char *name, void *host, uint64_t cap) {
    if (!g || !name || (!host && cap)) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_tensor_raw: NULL argument");
    return gg_guard([&] {
        const GgmlEntry &e = entry_of(g, name, "unknown tensor '");
        if (cap < e.len)
            gg_throw(FWHIP_ERR_INVALID, "fwhip_ggml_tensor_raw: buffer of " + std::to_string(cap) + " byte(s) for '" +
                                            name + "' of " + std::to_string(e.len));
        g->pread_exact(host, e.len, e.off, std::string("tensor '") + name + "' payload");
        return FWHIP_OK;
    });
}

// ---------------------------------------------------------------------------
// C ABI: device dequantization

extern "C" fwhip_status fwhip_dequant(fwhip_ctx *c, int32_t dtype, const void *raw_dev, uint64_t raw_bytes,
                                      int64_t n_elements, float *out_dev) {
    if (!c || (!raw_dev && raw_bytes) || (!out_dev && n_elements))
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_dequant: NULL argument");
    if (n_elements < 0) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dequant: negative element count");
    TypeInfo ti = type_info(dtype);
    if (!ti.qk) return fw_fail(FWHIP_ERR_UNSUPPORTED, "tensor element type " + std::to_string(dtype) + " is not supported");
    if (((uintptr_t)raw_dev & 3) || ((uintptr_t)out_dev & 3))
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_dequant: payload and output must be 4-byte aligned");
    return gg_guard([&] {
        uint64_t want = byte_len(dtype, (uint64_t)n_elements, "<device>");
        if (raw_bytes != want)
            gg_throw(FWHIP_ERR_INVALID, std::string("tensor '<device>' ") + ti.name + " byte length " +
                                            std::to_string(raw_bytes) + " != " + std::to_string(want));
        if (hipSetDevice(c->device) != hipSuccess) gg_throw(FWHIP_ERR_GENERIC, "fwhip_dequant: hipSetDevice failed");
        return dequant_launch(c, dtype, raw_dev, raw_bytes, out_dev, n_elements);
    });
}

// the payload of `e` decoded to f32 into out_dev (device), via pinned staging
static fwhip_status tensor_to_device_f32(fwhip_ctx *c, const fwhip_ggml *g, const std::string &name,
                                         const GgmlEntry &e, float *out_dev) {
    uint64_t n = n_elements(e);
    void *host = nullptr, *dev = nullptr;
    fwhip_status r = FWHIP_OK;
    if (hipHostMalloc(&host, e.len ? e.len : 4, hipHostMallocDefault) != hipSuccess)
        return fw_fail(FWHIP_ERR_GENERIC, "ggml: pinned staging allocation failed");
    r = gg_guard([&] {
        g->pread_exact(host, e.len, e.off, "tensor '" + name + "' payload");
        return FWHIP_OK;
    });
    if (r == FWHIP_OK && e.dtype == 0) {
        if (hipMemcpyAsync(out_dev, host, e.len, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
            hipStreamSynchronize(c->stream) != hipSuccess)
            r = fw_fail(FWHIP_ERR_GENERIC, "ggml: upload failed");
    } else if (r == FWHIP_OK) {
        if (hipMalloc(&dev, e.len ? e.len : 4) != hipSuccess ||
            hipMemcpyAsync(dev, host, e.len, hipMemcpyHostToDevice, c->stream) != hipSuccess)
            r = fw_fail(FWHIP_ERR_GENERIC, "ggml: device staging failed");
        if (r == FWHIP_OK) r = dequant_launch(c, e.dtype, dev, e.len, out_dev, (int64_t)n);
        if (r == FWHIP_OK && hipStreamSynchronize(c->stream) != hipSuccess)
            r = fw_fail(FWHIP_ERR_GENERIC, "ggml: dequantization failed");
    }
    if (dev) hipFree(dev);
    hipHostFree(host);
    return r;
}

extern "C" fwhip_status fwhip_ggml_tensor_f32(fwhip_ctx *c, const fwhip_ggml *g, const char *name, float *out_dev,
                                              int64_t n) {
    if (!c || !g || !name || !out_dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_ggml_tensor_f32: NULL argument");
    fwhip_status r = gg_guard([&] {
        const GgmlEntry &e = entry_of(g, name, "unknown tensor '");
        if ((uint64_t)n != n_elements(e))
            gg_throw(FWHIP_ERR_INVALID, std::string("fwhip_ggml_tensor_f32: '") + name + "' has " +
                                            std::to_string(n_elements(e)) + " elements, not " + std::to_string(n));
        if ((uintptr_t)out_dev & 3) gg_throw(FWHIP_ERR_INVALID, "fwhip_ggml_tensor_f32: output must be 4-byte aligned");
        return FWHIP_OK;
    });
    if (r != FWHIP_OK) return r;
    GG_HIP(hipSetDevice(c->device));
    return tensor_to_device_f32(c, g, name, g->tensors.at(name), out_dev);
}

// ---------------------------------------------------------------------------
// model loads

namespace {

struct Loader {
    fwhip_ctx *c;
    const fwhip_ggml *g;
    const char *side; // "encoder" / "decoder"
    std::vector<std::vector<float>> f32s;
    std::vector<std::vector<uint16_t>> h16s;

    const GgmlEntry &get(const std::string &name) { return entry_of(g, name.c_str(), "unknown tensor '"); }

    void check_cancel() {
        if (c->cancel.exchange(0)) gg_throw(FWHIP_ERR_CANCELLED, "cancelled");
    }

    // tensor_f32 on the host side of the boundary (any stored type)
    std::vector<float> &values(const std::string &name, const GgmlEntry &e) {
        uint64_t n = n_elements(e);
        f32s.emplace_back(n);
        std::vector<float> &v = f32s.back();
        if (e.dtype == 0) {
            g->pread_exact(v.data(), e.len, e.off, "tensor '" + name + "' payload");
        } else if (e.dtype == 1) {
            std::vector<uint16_t> h(n);
            g->pread_exact(h.data(), e.len, e.off, "tensor '" + name + "' payload");
            for (uint64_t i = 0; i < n; i++) v[i] = fw_host_h2f(h[i]);
        } else {
            float *dev = nullptr;
            if (hipMalloc(&dev, 4 * (n ? n : 1)) != hipSuccess) gg_throw(FWHIP_ERR_GENERIC, "ggml: device allocation failed");
            fwhip_status r = tensor_to_device_f32(c, g, name, e, dev);
            if (r == FWHIP_OK && hipMemcpy(v.data(), dev, 4 * n, hipMemcpyDeviceToHost) != hipSuccess)
                r = fw_fail(FWHIP_ERR_GENERIC, "ggml: download failed");
            hipFree(dev);
            if (r != FWHIP_OK) gg_throw(r, fwhip_last_error());
        }
        return v;
    }

    // a 1-D vector: encoder load_vec accepts [len] and [len, 1, ...]
    // (encoder.rs:387-399), decoder load_vec exactly [len] (decoder.rs:573-579)
    const float *vec(const std::string &name, uint64_t len) {
        const GgmlEntry &e = get(name);
        bool enc = side[0] == 'e';
        bool ok = enc ? (n_elements(e) == len && e.shape[0] == len) : (e.shape.size() == 1 && e.shape[0] == len);
        if (enc)
            for (size_t i = 1; ok && i < e.shape.size(); i++) ok = e.shape[i] == 1;
        if (!ok) {
            if (enc)
                gg_throw(FWHIP_ERR_INVALID, "encoder tensor '" + name + "' has shape " + fmt_shape(e.shape) +
                                                ", expected a length-" + std::to_string(len) + " vector");
            gg_throw(FWHIP_ERR_INVALID,
                     "decoder tensor '" + name + "' shape " + fmt_shape(e.shape) + " != expected [" + std::to_string(len) + "]");
        }
        return values(name, e).data();
    }

    // a shaped f32 tensor (encoder load_shaped, decoder tensor_shaped)
    const float *mat(const std::string &name, std::vector<uint64_t> want) {
        const GgmlEntry &e = get(name);
        if (e.shape != want) {
            if (side[0] == 'e')
                gg_throw(FWHIP_ERR_INVALID,
                         "encoder tensor '" + name + "' has shape " + fmt_shape(e.shape) + ", expected " + fmt_shape(want));
            gg_throw(FWHIP_ERR_INVALID,
                     "decoder tensor '" + name + "' shape " + fmt_shape(e.shape) + " != expected " + fmt_shape(want));
        }
        return values(name, e).data();
    }

    // a weight the GPU arms take as binary16 bits
    const uint16_t *w16(const std::string &name, std::vector<uint64_t> want, bool need_f16_storage) {
        const GgmlEntry &e = get(name);
        if (e.shape != want) {
            if (side[0] == 'e')
                gg_throw(FWHIP_ERR_INVALID,
                         "encoder tensor '" + name + "' has shape " + fmt_shape(e.shape) + ", expected " + fmt_shape(want));
            gg_throw(FWHIP_ERR_INVALID, std::string("decoder ") + (e.dtype == 1 ? "f16 " : "") + "tensor '" + name +
                                            "' shape " + fmt_shape(e.shape) + " != expected " + fmt_shape(want));
        }
        uint64_t n = n_elements(e);
        h16s.emplace_back(n);
        std::vector<uint16_t> &h = h16s.back();
        if (e.dtype == 1) {
            g->pread_exact(h.data(), e.len, e.off, "tensor '" + name + "' payload");
            return h.data();
        }
        if (need_f16_storage)
            gg_throw(FWHIP_ERR_UNSUPPORTED, std::string("cpu:ggml-") + type_info(e.dtype).name + "-linear: " + side +
                                                " tensor '" + name + "' is stored as " + type_info(e.dtype).name +
                                                "; the GPU decoder arms are the reference's f16-stored arms");
        // another stored type: accepted when every value is a binary16 value
        float *dev = nullptr;
        uint16_t *d16 = nullptr;
        int *bad = nullptr;
        fwhip_status r = FWHIP_OK;
        if (hipMalloc(&dev, 4 * n) != hipSuccess || hipMalloc(&d16, 2 * n) != hipSuccess ||
            hipMalloc(&bad, sizeof(int)) != hipSuccess || hipMemsetAsync(bad, 0, sizeof(int), c->stream) != hipSuccess)
            r = fw_fail(FWHIP_ERR_GENERIC, "ggml: device allocation failed");
        if (r == FWHIP_OK) r = tensor_to_device_f32(c, g, name, e, dev);
        int flag = 0;
        if (r == FWHIP_OK) {
            int grid = (int)((n + 255) / 256 < (uint64_t)c->n_cu * 8 ? (n + 255) / 256 : (uint64_t)c->n_cu * 8);
            hipLaunchKernelGGL(k_f16_exact, dim3(grid > 0 ? grid : 1), dim3(256), 0, c->stream, dev, d16, (int64_t)n, bad);
            if (hipMemcpyAsync(h.data(), d16, 2 * n, hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
                hipMemcpyAsync(&flag, bad, sizeof(int), hipMemcpyDeviceToHost, c->stream) != hipSuccess ||
                hipStreamSynchronize(c->stream) != hipSuccess)
                r = fw_fail(FWHIP_ERR_GENERIC, "ggml: f16 conversion failed");
        }
        if (dev) hipFree(dev);
        if (d16) hipFree(d16);
        if (bad) hipFree(bad);
        if (r != FWHIP_OK) gg_throw(r, fwhip_last_error());
        if (flag)
            gg_throw(FWHIP_ERR_UNSUPPORTED, std::string("cpu:ggml-") + type_info(e.dtype).name + "-linear: " + side +
                                                " tensor '" + name + "' is stored as " + type_info(e.dtype).name +
                                                " with values that are not binary16; the GPU arms compute with "
                                                "binary16 weights");
        return h.data();
    }
};

static fwhip_hparams hp_of(const fwhip_ggml *g) {
    fwhip_hparams h;
    h.n_vocab = g->hp[0];
    h.n_audio_ctx = g->hp[1];
    h.n_audio_state = g->hp[2];
    h.n_audio_head = g->hp[3];
    h.n_audio_layer = g->hp[4];
    h.n_text_ctx = g->hp[5];
    h.n_text_state = g->hp[6];
    h.n_text_head = g->hp[7];
    h.n_text_layer = g->hp[8];
    h.n_mels = g->hp[9];
    return h;
}

static uint64_t positive(int32_t v, const char *what) {
    if (v <= 0)
        gg_throw(FWHIP_ERR_INVALID,
                 std::string("encoder hparam '") + what + "' must be positive, got " + std::to_string(v));
    return (uint64_t)v;
}

} // namespace

// EncoderWeights::from_ggml (encoder.rs:764-1029): tensors in the reference's
// order, shapes checked with its messages, then fwhip_encoder_load
extern "C" fwhip_status fwhip_encoder_load_ggml(fwhip_ctx *c, const fwhip_ggml *g, int32_t precision,
                                                fwhip_encoder **out) {
    if (!c || !g || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_load_ggml: NULL argument");
    *out = nullptr;
    if (hipSetDevice(c->device) != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, "hipSetDevice failed");
    Loader L{c, g, "encoder", {}, {}};
    fwhip_encoder_weights w{};
    std::vector<fwhip_enc_layer> layers;
    fwhip_status r = gg_guard([&] {
        w.hp = hp_of(g);
        uint64_t n_mels = positive(g->hp[9], "n_mels"), d = positive(g->hp[2], "n_audio_state");
        uint64_t nh = positive(g->hp[3], "n_audio_head"), nl = positive(g->hp[4], "n_audio_layer");
        uint64_t nctx = positive(g->hp[1], "n_audio_ctx");
        if (d % nh)
            gg_throw(FWHIP_ERR_INVALID, "encoder: n_audio_head " + std::to_string(nh) + " does not divide n_audio_state " +
                                            std::to_string(d));
        uint64_t dff = 4 * d;
        w.conv1_w = L.w16("encoder.conv1.weight", {d, n_mels, 3}, false);
        w.conv1_b = L.vec("encoder.conv1.bias", d);
        w.conv2_w = L.w16("encoder.conv2.weight", {d, d, 3}, false);
        w.conv2_b = L.vec("encoder.conv2.bias", d);
        w.pos_emb = L.mat("encoder.positional_embedding", {nctx, d});
        layers.resize(nl);
        for (uint64_t i = 0; i < nl; i++) {
            L.check_cancel();
            std::string p = "encoder.blocks." + std::to_string(i) + ".";
            fwhip_enc_layer &l = layers[i];
            l.q_w = L.w16(p + "attn.query.weight", {d, d}, false);
            l.k_w = L.w16(p + "attn.key.weight", {d, d}, false);
            l.v_w = L.w16(p + "attn.value.weight", {d, d}, false);
            l.o_w = L.w16(p + "attn.out.weight", {d, d}, false);
            l.fc1_w = L.w16(p + "mlp.0.weight", {dff, d}, false);
            l.fc2_w = L.w16(p + "mlp.2.weight", {d, dff}, false);
            l.attn_ln_w = L.vec(p + "attn_ln.weight", d);
            l.attn_ln_b = L.vec(p + "attn_ln.bias", d);
            l.q_b = L.vec(p + "attn.query.bias", d);
            l.v_b = L.vec(p + "attn.value.bias", d);
            l.o_b = L.vec(p + "attn.out.bias", d);
            l.mlp_ln_w = L.vec(p + "mlp_ln.weight", d);
            l.mlp_ln_b = L.vec(p + "mlp_ln.bias", d);
            l.fc1_b = L.vec(p + "mlp.0.bias", dff);
            l.fc2_b = L.vec(p + "mlp.2.bias", d);
        }
        w.layers = layers.data();
        w.ln_post_w = L.vec("encoder.ln_post.weight", d);
        w.ln_post_b = L.vec("encoder.ln_post.bias", d);
        L.check_cancel();
        return FWHIP_OK;
    });
    if (r != FWHIP_OK) return r;
    return fwhip_encoder_load(c, &w, precision, out);
}

// DecoderWeights::from_ggml (decoder.rs:752-932)
extern "C" fwhip_status fwhip_decoder_load_ggml(fwhip_ctx *c, const fwhip_ggml *g, int32_t arm, fwhip_decoder **out) {
    if (!c || !g || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_decoder_load_ggml: NULL argument");
    *out = nullptr;
    if (hipSetDevice(c->device) != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, "hipSetDevice failed");
    Loader L{c, g, "decoder", {}, {}};
    fwhip_decoder_weights w{};
    std::vector<fwhip_dec_layer> layers;
    fwhip_status r = gg_guard([&] {
        w.hp = hp_of(g);
        const char *names[] = {"n_text_state", "n_text_head", "n_text_layer", "n_vocab", "n_text_ctx"};
        int32_t vals[] = {g->hp[6], g->hp[7], g->hp[8], g->hp[0], g->hp[5]};
        for (int i = 0; i < 5; i++)
            if (vals[i] < 0) gg_throw(FWHIP_ERR_INVALID, std::string("negative ") + names[i]);
        uint64_t d = (uint64_t)g->hp[6], nh = (uint64_t)g->hp[7], nl = (uint64_t)g->hp[8];
        uint64_t nv = (uint64_t)g->hp[0], nctx = (uint64_t)g->hp[5];
        if (nh == 0 || d % nh)
            gg_throw(FWHIP_ERR_INVALID,
                     "n_text_head " + std::to_string(nh) + " must divide n_text_state " + std::to_string(d));
        w.tok_emb = L.w16("decoder.token_embedding.weight", {nv, d}, true);
        w.pos_emb = L.mat("decoder.positional_embedding", {nctx, d});
        w.ln_w = L.vec("decoder.ln.weight", d);
        w.ln_b = L.vec("decoder.ln.bias", d);
        uint64_t dff = 4 * d;
        layers.resize(nl);
        for (uint64_t i = 0; i < nl; i++) {
            L.check_cancel();
            std::string p = "decoder.blocks." + std::to_string(i) + ".";
            fwhip_dec_layer &l = layers[i];
            l.attn_ln_w = L.vec(p + "attn_ln.weight", d);
            l.attn_ln_b = L.vec(p + "attn_ln.bias", d);
            l.q_w = L.w16(p + "attn.query.weight", {d, d}, true);
            l.q_b = L.vec(p + "attn.query.bias", d);
            l.k_w = L.w16(p + "attn.key.weight", {d, d}, true);
            l.v_w = L.w16(p + "attn.value.weight", {d, d}, true);
            l.v_b = L.vec(p + "attn.value.bias", d);
            l.o_w = L.w16(p + "attn.out.weight", {d, d}, true);
            l.o_b = L.vec(p + "attn.out.bias", d);
            l.cross_ln_w = L.vec(p + "cross_attn_ln.weight", d);
            l.cross_ln_b = L.vec(p + "cross_attn_ln.bias", d);
            l.cq_w = L.w16(p + "cross_attn.query.weight", {d, d}, true);
            l.cq_b = L.vec(p + "cross_attn.query.bias", d);
            l.ck_w = L.w16(p + "cross_attn.key.weight", {d, d}, true);
            l.cv_w = L.w16(p + "cross_attn.value.weight", {d, d}, true);
            l.cv_b = L.vec(p + "cross_attn.value.bias", d);
            l.co_w = L.w16(p + "cross_attn.out.weight", {d, d}, true);
            l.co_b = L.vec(p + "cross_attn.out.bias", d);
            l.mlp_ln_w = L.vec(p + "mlp_ln.weight", d);
            l.mlp_ln_b = L.vec(p + "mlp_ln.bias", d);
            l.fc1_w = L.w16(p + "mlp.0.weight", {dff, d}, true);
            l.fc1_b = L.vec(p + "mlp.0.bias", dff);
            l.fc2_w = L.w16(p + "mlp.2.weight", {d, dff}, true);
            l.fc2_b = L.vec(p + "mlp.2.bias", d);
        }
        w.layers = layers.data();
        L.check_cancel();
        return FWHIP_OK;
    });
    if (r != FWHIP_OK) return r;
    return fwhip_decoder_load(c, &w, arm, out);
}
