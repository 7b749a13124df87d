// mxh_gguf.cpp — GGUF reader / synthetic writer / row quantizers (host C++).
#include "mxh_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>

namespace mxh {

namespace {

struct BlockInfo {
    int elems, bytes;
};

BlockInfo block_info(int type) {
    switch (type) {
    case 0: return {1, 4};
    case 1: return {1, 2};
    case 6: return {32, 22};
    case 8: return {32, 34};
    case 12: return {256, 144};
    case 13: return {256, 176};
    case 14: return {256, 210};
    case 41: return {1, 1};  // one byte per element, the reference's reading
    }
    return {0, 0};
}

class Cursor {
public:
    Cursor(const uint8_t* p, size_t n) : p_(p), n_(n) {}
    bool ok() const { return ok_; }
    size_t pos() const { return pos_; }
    uint64_t u(int bytes) {
        if (pos_ + (size_t)bytes > n_) {
            ok_ = false;
            return 0;
        }
        uint64_t v = 0;
        for (int i = 0; i < bytes; ++i) v |= (uint64_t)p_[pos_ + i] << (8 * i);
        pos_ += (size_t)bytes;
        return v;
    }
    std::string str() {
        const uint64_t len = u(8);
        if (!ok_ || len > n_ - pos_) {
            ok_ = false;
            return {};
        }
        std::string s((const char*)p_ + pos_, (size_t)len);
        pos_ += (size_t)len;
        return s;
    }
    void skip(size_t n) {
        if (n > n_ - pos_) ok_ = false;
        else pos_ += n;
    }

private:
    const uint8_t* p_;
    size_t n_;
    size_t pos_ = 0;
    bool ok_ = true;
};

int scalar_size(uint32_t t) {
    switch (t) {
    case 0: case 1: case 7: return 1;
    case 2: case 3: return 2;
    case 4: case 5: case 6: return 4;
    case 10: case 11: case 12: return 8;
    }
    return -1;
}

double read_scalar(Cursor& c, uint32_t t) {
    switch (t) {
    case 0: return (double)(uint8_t)c.u(1);
    case 1: return (double)(int8_t)c.u(1);
    case 2: return (double)(uint16_t)c.u(2);
    case 3: return (double)(int16_t)c.u(2);
    case 4: return (double)(uint32_t)c.u(4);
    case 5: return (double)(int32_t)c.u(4);
    case 6: { uint32_t b = (uint32_t)c.u(4); float f; std::memcpy(&f, &b, 4); return f; }
    case 7: return (double)c.u(1);
    case 10: return (double)c.u(8);
    case 11: return (double)(int64_t)c.u(8);
    case 12: { uint64_t b = c.u(8); double f; std::memcpy(&f, &b, 8); return f; }
    }
    return 0.0;
}

// ---- fp16 encode (round to nearest even) ----
uint16_t f2h(float v) {
    uint32_t x;
    std::memcpy(&x, &v, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax < 0x38800000u) {
        // subnormal half: scale into integer units of 2^-24 and round
        const float mag = std::fabs(v) * 16777216.0f;  // exact (power-of-two scale)
        return (uint16_t)(sign | (uint32_t)std::nearbyint(mag));
    }
    uint32_t r = ((ax >> 23) - 112u) << 10 | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u, f = h & 1023u;
    float v;
    if (e == 0) v = std::ldexp((float)f, -24);
    else if (e == 31) v = f ? NAN : INFINITY;
    else v = std::ldexp((float)(f | 1024u), (int)e - 25);
    return s ? -v : v;
}

void put16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

int qround(float v, int lo, int hi) {
    const int r = (int)std::lrint(v);
    return r < lo ? lo : (r > hi ? hi : r);
}

// 8 sub-blocks of 32: affine codes in [0, qmax], 6-bit scale/offset packed
// in the ggml K-quant scale layout.
void quant_k_block(const float* v, int qmax, uint8_t* hdr16, int* codes) {
    float sc[8], off[8], smax = 0.f, omax = 0.f;
    for (int j = 0; j < 8; ++j) {
        const float* s = v + 32 * j;
        float lo = *std::min_element(s, s + 32), hi = *std::max_element(s, s + 32);
        lo = std::min(lo, 0.f);
        sc[j] = (hi - lo) / (float)qmax;
        off[j] = -lo;
        smax = std::max(smax, sc[j]);
        omax = std::max(omax, off[j]);
    }
    const uint16_t dh = f2h(smax / 63.f), mh = f2h(omax / 63.f);
    const float d = h2f(dh), dm = h2f(mh);
    int s6[8], m6[8];
    for (int j = 0; j < 8; ++j) {
        s6[j] = d > 0.f ? qround(sc[j] / d, 0, 63) : 0;
        m6[j] = dm > 0.f ? qround(off[j] / dm, 0, 63) : 0;
        const float ds = d * (float)s6[j], ms = dm * (float)m6[j];
        for (int i = 0; i < 32; ++i) codes[32 * j + i] = ds > 0.f ? qround((v[32 * j + i] + ms) / ds, 0, qmax) : 0;
    }
    put16(hdr16, dh);
    put16(hdr16 + 2, mh);
    uint8_t* s = hdr16 + 4;
    std::memset(s, 0, 12);
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)(s6[j] | ((s6[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)(m6[j] | ((m6[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((s6[j + 4] & 15) | ((m6[j + 4] & 15) << 4));
    }
}

// splitmix64 stream -> N(0, 1) by Box-Muller
struct Normal {
    uint64_t s;
    bool have = false;
    float spare = 0.f;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float operator()() {
        if (have) {
            have = false;
            return spare;
        }
        const uint64_t r = next();
        const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777217.0f);  // (0, 1]
        const float u2 = (float)((r >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
        const float rad = std::sqrt(-2.0f * std::log(u1));
        spare = rad * std::sin(6.2831853f * u2);
        have = true;
        return rad * std::cos(6.2831853f * u2);
    }
};

uint64_t mix(uint64_t a, uint64_t b) {
    uint64_t z = a ^ (b + 0x9E3779B97F4A7C15ull + (a << 6) + (a >> 2));
    z = (z ^ (z >> 31)) * 0xD6E8FEB86659FD93ull;
    return z ^ (z >> 32);
}

}  // namespace

size_t tensor_bytes(int type, int64_t rows, int64_t cols) {
    const BlockInfo b = block_info(type);
    if (!b.elems || rows < 0 || cols < 0 || cols % b.elems) return 0;
    size_t row = 0, total = 0;
    if (__builtin_mul_overflow((size_t)(cols / b.elems), (size_t)b.bytes, &row) ||
        __builtin_mul_overflow((size_t)rows, row, &total))
        return 0;
    return total;
}

void quantize_row(int type, const float* x, int64_t n, uint8_t* out) {
    if (type == 0) {
        std::memcpy(out, x, (size_t)n * 4);
    } else if (type == 41) {
        // byte values, for synthetic files: small non-negative integers
        for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)qround(x[i] * 64.f + 2.f, 0, 255);
    } else if (type == 1) {
        for (int64_t i = 0; i < n; ++i) put16(out + 2 * i, f2h(x[i]));
    } else if (type == 8) {
        for (int64_t b = 0; b < n / 32; ++b) {
            const float* v = x + 32 * b;
            uint8_t* o = out + 34 * b;
            float amax = 0.f;
            for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(v[i]));
            const uint16_t dh = f2h(amax / 127.f);
            const float d = h2f(dh);
            put16(o, dh);
            for (int i = 0; i < 32; ++i) o[2 + i] = (uint8_t)(int8_t)(d > 0.f ? qround(v[i] / d, -127, 127) : 0);
        }
    } else if (type == 12 || type == 13) {
        const int bb = type == 12 ? 144 : 176;
        int codes[256];
        for (int64_t b = 0; b < n / 256; ++b) {
            uint8_t* o = out + (size_t)bb * b;
            quant_k_block(x + 256 * b, type == 12 ? 15 : 31, o, codes);
            uint8_t* qs = o + (type == 12 ? 16 : 48);
            if (type == 13) std::memset(o + 16, 0, 32);
            for (int g = 0; g < 4; ++g)
                for (int i = 0; i < 32; ++i) {
                    const int a = codes[64 * g + i], c = codes[64 * g + 32 + i];
                    qs[32 * g + i] = (uint8_t)((a & 15) | ((c & 15) << 4));
                    if (type == 13) o[16 + i] |= (uint8_t)(((a >> 4) << (2 * g)) | ((c >> 4) << (2 * g + 1)));
                }
        }
    } else if (type == 14) {
        // Q6_K: per 16 elements a signed 8-bit scale (amax / 31 over d, d the
        // largest of them / 127), codes q + 32 in [0, 63]; layout as the
        // reference's gguf_dequant_q6_k reads it (gguf_reader.cpp:905-1008)
        for (int64_t b = 0; b < n / 256; ++b) {
            const float* v = x + 256 * b;
            uint8_t* o = out + (size_t)210 * b;
            float sf[16], smax = 0.f;
            for (int j = 0; j < 16; ++j) {
                float amax = 0.f;
                for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(v[16 * j + i]));
                sf[j] = amax / 31.f;
                smax = std::max(smax, sf[j]);
            }
            const uint16_t dh = f2h(smax / 127.f);
            const float d = h2f(dh);
            int q[256];
            for (int j = 0; j < 16; ++j) {
                const int sc = d > 0.f ? qround(sf[j] / d, -128, 127) : 0;
                o[192 + j] = (uint8_t)(int8_t)sc;
                const float ds = d * (float)sc;
                for (int i = 0; i < 16; ++i) q[16 * j + i] = (ds != 0.f ? qround(v[16 * j + i] / ds, -32, 31) : 0) + 32;
            }
            std::memset(o, 0, 192);
            for (int h = 0; h < 2; ++h)
                for (int l = 0; l < 32; ++l) {
                    const int* qq = q + 128 * h + l;
                    o[64 * h + l] = (uint8_t)((qq[0] & 15) | ((qq[64] & 15) << 4));
                    o[64 * h + 32 + l] = (uint8_t)((qq[32] & 15) | ((qq[96] & 15) << 4));
                    o[128 + 32 * h + l] =
                        (uint8_t)((qq[0] >> 4) | ((qq[32] >> 4) << 2) | ((qq[64] >> 4) << 4) | ((qq[96] >> 4) << 6));
                }
            put16(o + 208, dh);
        }
    } else if (type == 6) {
        for (int64_t b = 0; b < n / 32; ++b) {
            const float* v = x + 32 * b;
            uint8_t* o = out + 22 * b;
            float amax = 0.f, mx = 0.f;
            for (int i = 0; i < 32; ++i)
                if (std::fabs(v[i]) > amax) { amax = std::fabs(v[i]); mx = v[i]; }
            const uint16_t dh = f2h(mx / -16.f);
            const float d = h2f(dh);
            uint32_t qh = 0;
            std::memset(o + 6, 0, 16);
            for (int i = 0; i < 32; ++i) {
                const int q = d != 0.f ? qround(v[i] / d + 16.f, 0, 31) : 16;
                o[6 + (i & 15)] |= (uint8_t)((q & 15) << (i < 16 ? 0 : 4));
                qh |= (uint32_t)(q >> 4) << i;
            }
            put16(o, dh);
            std::memcpy(o + 2, &qh, 4);
        }
    }
}

GgufFile::~GgufFile() {
    if (map_) munmap(map_, size_);
}

bool GgufFile::open(const std::string& path, std::string* err) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) {
        *err = "cannot open " + path;
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        *err = "cannot stat " + path;
        return false;
    }
    void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
        *err = "mmap failed for " + path;
        return false;
    }
    map_ = m;
    size_ = (size_t)st.st_size;
    const uint8_t* base = (const uint8_t*)m;
    Cursor c(base, size_);
    if (c.u(4) != 0x46554747u) {
        *err = "not a GGUF file";
        return false;
    }
    const uint32_t version = (uint32_t)c.u(4);
    if (version < 2 || version > 3) {
        *err = "unsupported GGUF version " + std::to_string(version);
        return false;
    }
    const uint64_t n_tensors = c.u(8), n_kv = c.u(8);
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < n_kv && c.ok(); ++i) {
        const std::string key = c.str();
        const uint32_t t = (uint32_t)c.u(4);
        if (!c.ok()) break;  // reported as a truncated header below
        if (t == 8) {
            strs_[key] = c.str();
        } else if (t == 9) {
            const uint32_t et = (uint32_t)c.u(4);
            const uint64_t cnt = c.u(8);
            for (uint64_t e = 0; e < cnt && c.ok(); ++e) {
                if (et == 8) (void)c.str();
                else if (scalar_size(et) > 0) c.skip((size_t)scalar_size(et));
                else { *err = "bad array element type"; return false; }
            }
        } else if (scalar_size(t) > 0) {
            nums_[key] = read_scalar(c, t);
            if (key == "general.alignment") alignment = (uint64_t)nums_[key];
        } else {
            *err = "bad metadata type for " + key;
            return false;
        }
    }
    auto it = strs_.find("general.architecture");
    arch_ = it != strs_.end() ? it->second : "";
    if (!c.ok()) {
        *err = "truncated GGUF header";
        return false;
    }
    // a directory entry takes at least 32 bytes (name length, rank, one
    // dimension, type, offset): a count beyond what the file can hold is corrupt
    if (n_tensors > (size_ - c.pos()) / 32) {
        *err = "tensor count exceeds the file";
        return false;
    }
    tensors_.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors && c.ok(); ++i) {
        GgufTensor& t = tensors_[(size_t)i];
        t.name = c.str();
        t.n_dims = (int)c.u(4);
        if (t.n_dims < 1 || t.n_dims > 4) { *err = "bad tensor rank for " + t.name; return false; }
        for (int d = 0; d < t.n_dims; ++d) {
            const uint64_t ne = c.u(8);
            if (ne > (uint64_t)INT64_MAX) { *err = "bad dimension for " + t.name; return false; }
            t.ne[d] = (int64_t)ne;
        }
        t.type = (int)c.u(4);
        t.offset = c.u(8);
    }
    if (!c.ok()) {
        *err = "truncated GGUF header";
        return false;
    }
    if (alignment == 0 || (alignment & (alignment - 1)) || alignment > (1u << 20)) { *err = "bad alignment"; return false; }
    const size_t data0 = (c.pos() + alignment - 1) / alignment * alignment;
    if (data0 > size_) { *err = "tensor data starts past end of file"; return false; }
    for (size_t i = 0; i < tensors_.size(); ++i) {
        GgufTensor& t = tensors_[i];
        int64_t rows = 1;
        bool overflow = false;
        for (int d = 1; d < t.n_dims; ++d) overflow |= __builtin_mul_overflow(rows, t.ne[d], &rows);
        if (overflow) { *err = "tensor " + t.name + " has too many elements"; return false; }
        t.nbytes = tensor_bytes(t.type, rows, t.ne[0]);
        if (block_info(t.type).elems == 0) continue;  // unknown type: not addressable
        if (t.nbytes == 0 && rows > 0 && t.ne[0] > 0) {
            *err = "tensor " + t.name + " is not a whole number of blocks";
            return false;
        }
        // offset, then size, against the bytes left (no sum that can wrap)
        if (t.offset > size_ - data0 || t.nbytes > size_ - data0 - t.offset) {
            *err = "tensor " + t.name + " extends past end of file";
            return false;
        }
        t.data = base + data0 + t.offset;
        index_[t.name] = i;
    }
    return true;
}

const GgufTensor* GgufFile::find(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

double GgufFile::arch_num(const std::string& suffix, double def) const {
    auto it = nums_.find(arch_ + "." + suffix);
    return it == nums_.end() ? def : it->second;
}

// ---- synthetic writer ----

namespace {

struct Plan {
    std::string name;
    int type;
    int64_t rows, cols;  // cols = ne[0]
    bool norm;
    uint64_t offset;
};

void w_str(std::string& b, const std::string& s) {
    const uint64_t n = s.size();
    b.append((const char*)&n, 8);
    b += s;
}
void w_u32(std::string& b, uint32_t v) { b.append((const char*)&v, 4); }
void w_u64(std::string& b, uint64_t v) { b.append((const char*)&v, 8); }
void kv_u32(std::string& b, const std::string& k, uint32_t v) { w_str(b, k); w_u32(b, 4); w_u32(b, v); }
void kv_f32(std::string& b, const std::string& k, float v) {
    w_str(b, k);
    w_u32(b, 6);
    b.append((const char*)&v, 4);
}
void kv_str(std::string& b, const std::string& k, const std::string& v) { w_str(b, k); w_u32(b, 8); w_str(b, v); }

}  // namespace

bool write_synthetic_gguf(const std::string& path, const SynthArch& a, uint64_t seed, int threads, std::string* err) {
    const int qd = a.n_head * a.head_dim, kvd = a.n_head_kv * a.head_dim;
    std::vector<Plan> plan;
    auto add = [&](const std::string& n, int t, int64_t rows, int64_t cols) { plan.push_back({n, t, rows, cols, false, 0}); };
    auto norm = [&](const std::string& n, int64_t len) { plan.push_back({n, 0, 1, len, true, 0}); };
    if (!a.tied) add("output.weight", a.out_type, a.n_vocab, a.n_embd);
    add("token_embd.weight", a.embd_type, a.n_vocab, a.n_embd);
    norm("output_norm.weight", a.n_embd);
    for (int l = 0; l < a.n_layer; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        norm(p + "attn_norm.weight", a.n_embd);
        add(p + "attn_q.weight", a.wtype, qd, a.n_embd);
        add(p + "attn_k.weight", a.wtype, kvd, a.n_embd);
        add(p + "attn_v.weight", a.attn_v_type >= 0 ? a.attn_v_type : a.wtype, kvd, a.n_embd);
        if (a.qk_norm) {
            norm(p + "attn_q_norm.weight", a.head_dim);
            norm(p + "attn_k_norm.weight", a.head_dim);
        }
        add(p + "attn_output.weight", a.wtype, a.n_embd, qd);
        norm(p + "ffn_norm.weight", a.n_embd);
        add(p + "ffn_gate.weight", a.wtype, a.n_ff, a.n_embd);
        add(p + "ffn_up.weight", a.wtype, a.n_ff, a.n_embd);
        add(p + "ffn_down.weight", a.ffn_down_type >= 0 ? a.ffn_down_type : a.wtype, a.n_embd, a.n_ff);
    }
    const uint64_t align = 32;
    uint64_t off = 0;
    for (Plan& p : plan) {
        const size_t nb = tensor_bytes(p.type, p.rows, p.cols);
        if (!nb) { *err = "shape of " + p.name + " is not a whole number of blocks"; return false; }
        off = (off + align - 1) / align * align;
        p.offset = off;
        off += nb;
    }
    const std::string ar = a.arch;
    std::string h;
    w_u32(h, 0x46554747u);
    w_u32(h, 3);
    w_u64(h, plan.size());
    w_u64(h, 14);
    kv_u32(h, "general.alignment", (uint32_t)align);
    kv_str(h, "general.architecture", ar);
    kv_str(h, "general.name", "synthetic-" + ar + "-seed" + std::to_string(seed));
    kv_u32(h, ar + ".block_count", (uint32_t)a.n_layer);
    kv_u32(h, ar + ".context_length", (uint32_t)a.ctx);
    kv_u32(h, ar + ".embedding_length", (uint32_t)a.n_embd);
    kv_u32(h, ar + ".feed_forward_length", (uint32_t)a.n_ff);
    kv_u32(h, ar + ".attention.head_count", (uint32_t)a.n_head);
    kv_u32(h, ar + ".attention.head_count_kv", (uint32_t)a.n_head_kv);
    kv_u32(h, ar + ".attention.key_length", (uint32_t)a.head_dim);
    kv_u32(h, ar + ".attention.value_length", (uint32_t)a.head_dim);
    kv_f32(h, ar + ".rope.freq_base", a.rope_theta);
    kv_f32(h, ar + ".attention.layer_norm_rms_epsilon", a.eps);
    kv_u32(h, ar + ".vocab_size", (uint32_t)a.n_vocab);
    for (const Plan& p : plan) {
        w_str(h, p.name);
        const bool two_d = !p.norm;
        w_u32(h, two_d ? 2 : 1);
        w_u64(h, (uint64_t)p.cols);
        if (two_d) w_u64(h, (uint64_t)p.rows);
        w_u32(h, (uint32_t)p.type);
        w_u64(h, p.offset);
    }
    h.resize((h.size() + align - 1) / align * align, '\0');
    const uint64_t data0 = h.size();

    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) { *err = "cannot create " + path; return false; }
    const bool head_ok = std::fwrite(h.data(), 1, h.size(), f) == h.size();
    std::fclose(f);
    if (!head_ok) { *err = "write failed"; return false; }
    const int fd = ::open(path.c_str(), O_WRONLY);
    if (fd < 0 || ftruncate(fd, (off_t)(data0 + off)) != 0) {
        if (fd >= 0) ::close(fd);
        *err = "cannot size " + path;
        return false;
    }
    if (threads <= 0) threads = (int)std::max(1u, std::thread::hardware_concurrency());
    bool ok = true;
    for (size_t ti = 0; ti < plan.size() && ok; ++ti) {
        const Plan& p = plan[ti];
        const size_t rb = tensor_bytes(p.type, 1, p.cols);
        std::vector<uint8_t> buf(rb * (size_t)p.rows);
        const uint64_t tseed = mix(seed, ti + 1);
        auto work = [&](int64_t r0, int64_t r1) {
            std::vector<float> row((size_t)p.cols);
            for (int64_t r = r0; r < r1; ++r) {
                Normal g{mix(tseed, (uint64_t)r)};
                if (p.norm)
                    for (auto& v : row) v = 1.0f + 0.02f * g();
                else
                    for (auto& v : row) v = 0.02f * g();
                quantize_row(p.type, row.data(), p.cols, buf.data() + (size_t)r * rb);
            }
        };
        const int nt = (int)std::min<int64_t>(threads, p.rows);
        std::vector<std::thread> pool;
        for (int t = 0; t < nt; ++t) pool.emplace_back(work, p.rows * t / nt, p.rows * (t + 1) / nt);
        for (auto& th : pool) th.join();
        size_t done = 0;
        while (done < buf.size()) {
            const ssize_t w = pwrite(fd, buf.data() + done, buf.size() - done, (off_t)(data0 + p.offset + done));
            if (w <= 0) { ok = false; break; }
            done += (size_t)w;
        }
    }
    ::close(fd);
    if (!ok) *err = "write failed for " + path;
    return ok;
}

}  // namespace mxh
