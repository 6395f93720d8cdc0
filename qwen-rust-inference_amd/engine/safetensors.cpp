// Checkpoint reader for the real Qwen3.5 weights: a streaming safetensors
// reader with SHA-256 verification (the reference's read_checkpoint_kept,
// src/weights.rs:364-466, and decode_tensor, 168-186). One sequential pass over
// the file: every byte goes through SHA-256 while each kept tensor is read into
// its own buffer (BF16 kept as bits, F32 decoded); ignored tensors are hashed
// and skipped. The header checks are the safetensors format's: an 8-byte
// little-endian header length, a JSON object of {name: {dtype, shape,
// data_offsets}} (plus an optional "__metadata__"), offsets contiguous from 0,
// each size = product(shape) x dtype size, and the data ending exactly at the
// end of the file. Nothing is handed out unless the whole file hashes to the
// expected digest (when one is given).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/qwen_engine.h"

namespace {

// ---------------------------------------------------------------- SHA-256 (FIPS 180-4)
class Sha256 {
public:
    Sha256() { reset(); }
    void update(const uint8_t* p, size_t n) {
        total_ += n;
        while (n > 0) {
            const size_t k = std::min(n, size_t(64) - fill_);
            std::memcpy(block_ + fill_, p, k);
            fill_ += k;
            p += k;
            n -= k;
            if (fill_ == 64) {
                compress(block_);
                fill_ = 0;
            }
        }
    }
    std::string hex() {
        uint64_t bits = total_ * 8;
        const uint8_t one = 0x80, zero = 0;
        update(&one, 1);
        while (fill_ != 56) update(&zero, 1);
        uint8_t len[8];
        for (int i = 0; i < 8; ++i) len[i] = uint8_t(bits >> (56 - 8 * i));
        update(len, 8);
        char out[65];
        for (int i = 0; i < 8; ++i) std::snprintf(out + 8 * i, 9, "%08x", h_[i]);
        return std::string(out, 64);
    }

private:
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void reset() {
        static const uint32_t init[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                         0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
        std::memcpy(h_, init, sizeof h_);
        fill_ = 0;
        total_ = 0;
    }
    void compress(const uint8_t* b) {
        static const uint32_t k[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
            0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
            0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
            0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
            0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
            0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
            0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = uint32_t(b[4 * i]) << 24 | uint32_t(b[4 * i + 1]) << 16 | uint32_t(b[4 * i + 2]) << 8 | b[4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h_[0], bb = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], hh = h_[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
            const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & bb) ^ (a & c) ^ (bb & c));
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = bb;
            bb = a;
            a = t1 + t2;
        }
        h_[0] += a, h_[1] += bb, h_[2] += c, h_[3] += d, h_[4] += e, h_[5] += f, h_[6] += g, h_[7] += hh;
    }
    uint32_t h_[8];
    uint8_t block_[64];
    size_t fill_;
    uint64_t total_;
};

// ---------------------------------------------------------------- the header's JSON
struct Json {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    double number = 0;
    bool boolean = false;
    std::string text;
    std::vector<Json> items;
    std::vector<std::pair<std::string, Json>> members;
};

class Parser {
public:
    explicit Parser(const std::string& s) : s_(s) {}
    Json document() {
        Json v = value();
        space();
        if (i_ != s_.size()) fail("trailing characters");
        return v;
    }

private:
    [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("safetensors header: ") + what); }
    void space() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    char peek() {
        space();
        if (i_ >= s_.size()) fail("unexpected end");
        return s_[i_];
    }
    void expect(char c) {
        if (peek() != c) fail("unexpected character");
        ++i_;
    }
    Json value() {
        if (++depth_ > 64) fail("nesting too deep");
        Json v;
        const char c = peek();
        if (c == '{') {
            v.kind = Json::Object;
            ++i_;
            if (peek() == '}') {
                ++i_;
            } else {
                for (;;) {
                    std::string key = string();
                    expect(':');
                    v.members.emplace_back(std::move(key), value());
                    if (peek() == ',') {
                        ++i_;
                        continue;
                    }
                    expect('}');
                    break;
                }
            }
        } else if (c == '[') {
            v.kind = Json::Array;
            ++i_;
            if (peek() == ']') {
                ++i_;
            } else {
                for (;;) {
                    v.items.push_back(value());
                    if (peek() == ',') {
                        ++i_;
                        continue;
                    }
                    expect(']');
                    break;
                }
            }
        } else if (c == '"') {
            v.kind = Json::String;
            v.text = string();
        } else if (s_.compare(i_, 4, "true") == 0) {
            v.kind = Json::Bool, v.boolean = true, i_ += 4;
        } else if (s_.compare(i_, 5, "false") == 0) {
            v.kind = Json::Bool, i_ += 5;
        } else if (s_.compare(i_, 4, "null") == 0) {
            i_ += 4;
        } else if (c == '-' || (c >= '0' && c <= '9')) {
            v.kind = Json::Number;
            const size_t start = i_;
            while (i_ < s_.size() && std::strchr("+-0123456789.eE", s_[i_])) ++i_;
            v.text = s_.substr(start, i_ - start);
            v.number = std::strtod(v.text.c_str(), nullptr);
        } else {
            fail("bad value");
        }
        --depth_;
        return v;
    }
    static void utf8(std::string& out, uint32_t cp) {
        if (cp < 0x80) {
            out += char(cp);
        } else if (cp < 0x800) {
            out += char(0xc0 | (cp >> 6)), out += char(0x80 | (cp & 0x3f));
        } else if (cp < 0x10000) {
            out += char(0xe0 | (cp >> 12)), out += char(0x80 | ((cp >> 6) & 0x3f)), out += char(0x80 | (cp & 0x3f));
        } else {
            out += char(0xf0 | (cp >> 18)), out += char(0x80 | ((cp >> 12) & 0x3f));
            out += char(0x80 | ((cp >> 6) & 0x3f)), out += char(0x80 | (cp & 0x3f));
        }
    }
    uint32_t hex4() {
        if (i_ + 4 > s_.size()) fail("bad escape");
        uint32_t v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = s_[i_++];
            v <<= 4;
            if (c >= '0' && c <= '9') v |= uint32_t(c - '0');
            else if (c >= 'a' && c <= 'f') v |= uint32_t(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= uint32_t(c - 'A' + 10);
            else fail("bad escape");
        }
        return v;
    }
    std::string string() {
        expect('"');
        std::string out;
        for (;;) {
            if (i_ >= s_.size()) fail("unterminated string");
            const char c = s_[i_++];
            if (c == '"') return out;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i_ >= s_.size()) fail("bad escape");
            const char e = s_[i_++];
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\b'; break;
            case 'f': out += '\f'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                uint32_t cp = hex4();
                if (cp >= 0xd800 && cp < 0xdc00 && i_ + 6 <= s_.size() && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
                    i_ += 2;
                    const uint32_t lo = hex4();
                    cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                }
                utf8(out, cp);
                break;
            }
            default: fail("bad escape");
            }
        }
    }
    const std::string& s_;
    size_t i_ = 0;
    int depth_ = 0;
};

uint64_t whole(const Json& v, const char* what) {
    if (v.kind != Json::Number || v.number < 0 || v.number != std::floor(v.number) || v.number > 9.0e15)
        throw std::runtime_error(std::string("safetensors header: bad ") + what);
    return uint64_t(v.number);
}

struct Entry {
    std::string name;
    int dtype = 0;  // QE_ST_F32 / QE_ST_BF16
    std::vector<int64_t> shape;
    uint64_t begin = 0, end = 0;
    bool kept = false;
    std::vector<uint16_t> bits;  // BF16
    std::vector<float> values;   // F32
};

thread_local std::string g_st_error;

}  // namespace

struct QeSafetensors {
    std::vector<Entry> tensors;  // in data order
    std::string sha256;
    std::map<std::string, size_t> index;
};

extern "C" {

const char* qe_safetensors_error(void) { return g_st_error.c_str(); }

QeSafetensors* qe_safetensors_read(const char* path, const char* expected_sha256, const char* const* ignored,
                                   int64_t n_ignored) {
    FILE* f = nullptr;
    try {
        g_st_error.clear();
        f = std::fopen(path, "rb");
        if (!f) throw std::runtime_error(std::string("cannot open ") + path);
        if (std::fseek(f, 0, SEEK_END) != 0) throw std::runtime_error("cannot seek");
        const long length = std::ftell(f);
        std::rewind(f);
        Sha256 hash;
        auto read = [&](void* dst, size_t n) {
            if (n && std::fread(dst, 1, n, f) != n) throw std::runtime_error("safetensors: file truncated");
            hash.update(static_cast<const uint8_t*>(dst), n);
        };
        uint8_t len8[8];
        read(len8, 8);
        uint64_t n = 0;
        for (int i = 7; i >= 0; --i) n = n << 8 | len8[i];
        if (n > 100000000ull || n + 8 > uint64_t(length)) throw std::runtime_error("safetensors header length");
        std::string header(size_t(n), '\0');
        read(&header[0], size_t(n));
        const Json doc = Parser(header).document();
        if (doc.kind != Json::Object) throw std::runtime_error("safetensors header: not an object");
        auto out = std::make_unique<QeSafetensors>();
        for (const auto& m : doc.members) {
            if (m.first == "__metadata__") continue;
            const Json& v = m.second;
            const Json *dtype = nullptr, *shape = nullptr, *offsets = nullptr;
            for (const auto& f2 : v.members) {
                if (f2.first == "dtype") dtype = &f2.second;
                else if (f2.first == "shape") shape = &f2.second;
                else if (f2.first == "data_offsets") offsets = &f2.second;
            }
            if (v.kind != Json::Object || !dtype || !shape || !offsets || dtype->kind != Json::String ||
                shape->kind != Json::Array || offsets->kind != Json::Array || offsets->items.size() != 2)
                throw std::runtime_error("safetensors header: bad entry " + m.first);
            Entry e;
            e.name = m.first;
            if (dtype->text == "F32") e.dtype = QE_ST_F32;
            else if (dtype->text == "BF16") e.dtype = QE_ST_BF16;
            else e.dtype = -1;  // allowed only for ignored tensors
            for (const auto& d : shape->items) e.shape.push_back(int64_t(whole(d, "shape")));
            e.begin = whole(offsets->items[0], "offsets");
            e.end = whole(offsets->items[1], "offsets");
            const uint64_t size = dtype->text == "F32" ? 4 : dtype->text == "BF16" || dtype->text == "F16" ? 2
                                  : dtype->text == "F64" || dtype->text == "I64" ? 8
                                  : dtype->text == "I32" ? 4 : dtype->text == "I8" || dtype->text == "U8" || dtype->text == "BOOL" ? 1 : 0;
            if (size == 0) throw std::runtime_error("safetensors: unsupported dtype " + dtype->text + ": " + e.name);
            uint64_t bytes = size;
            for (int64_t d : e.shape) {
                if (d != 0 && bytes > UINT64_MAX / uint64_t(d)) throw std::runtime_error("safetensors offsets: " + e.name);
                bytes *= uint64_t(d);
            }
            if (e.end < e.begin || e.end - e.begin != bytes) throw std::runtime_error("safetensors offsets: " + e.name);
            e.kept = true;
            for (int64_t k = 0; k < n_ignored; ++k)
                if (ignored && ignored[k] && e.name == ignored[k]) e.kept = false;
            if (e.kept && e.dtype < 0) throw std::runtime_error("safetensors: unsupported dtype " + dtype->text + ": " + e.name);
            out->tensors.push_back(std::move(e));
        }
        std::sort(out->tensors.begin(), out->tensors.end(),
                  [](const Entry& a, const Entry& b) { return a.begin < b.begin; });
        uint64_t end = 0;
        for (const Entry& e : out->tensors) {
            if (e.begin != end) throw std::runtime_error("safetensors offsets: " + e.name);
            end = e.end;
        }
        if (end + 8 + n != uint64_t(length)) throw std::runtime_error("safetensors data length");
        std::vector<uint8_t> chunk(1 << 20);
        for (Entry& e : out->tensors) {
            uint64_t left = e.end - e.begin;
            if (!e.kept) {
                while (left > 0) {
                    const size_t k = size_t(std::min<uint64_t>(left, chunk.size()));
                    read(chunk.data(), k);
                    left -= k;
                }
                continue;
            }
            if (left == 0) throw std::runtime_error("empty tensor: " + e.name);
            if (e.dtype == QE_ST_BF16) {
                e.bits.resize(size_t(left / 2));
                read(e.bits.data(), size_t(left));  // little-endian words on this host
                for (uint16_t b : e.bits)
                    if ((b & 0x7f80) == 0x7f80) throw std::runtime_error("NaN/Inf detected: " + e.name);
            } else {
                e.values.resize(size_t(left / 4));
                read(e.values.data(), size_t(left));
                for (float v : e.values)
                    if (!std::isfinite(v)) throw std::runtime_error("NaN/Inf detected: " + e.name);
            }
        }
        std::fclose(f);
        f = nullptr;
        out->sha256 = hash.hex();
        if (expected_sha256 && out->sha256 != expected_sha256) throw std::runtime_error("checkpoint SHA-256 mismatch");
        for (size_t i = 0; i < out->tensors.size(); ++i) out->index[out->tensors[i].name] = i;
        return out.release();
    } catch (const std::exception& e) {
        if (f) std::fclose(f);
        g_st_error = e.what();
        return nullptr;
    }
}

void qe_safetensors_free(QeSafetensors* s) { delete s; }
const char* qe_safetensors_sha256(const QeSafetensors* s) { return s->sha256.c_str(); }
int64_t qe_safetensors_count(const QeSafetensors* s) { return int64_t(s->tensors.size()); }

int qe_safetensors_info(const QeSafetensors* s, int64_t i, const char** name, int* dtype, int* kept, int* ndim,
                        int64_t* shape) {
    if (i < 0 || size_t(i) >= s->tensors.size()) {
        g_st_error = "tensor index out of range";
        return -1;
    }
    const Entry& e = s->tensors[size_t(i)];
    *name = e.name.c_str();
    *dtype = e.dtype;
    *kept = e.kept ? 1 : 0;
    *ndim = int(e.shape.size());
    for (size_t d = 0; d < e.shape.size() && d < 8; ++d) shape[d] = e.shape[d];
    return 0;
}

// The tensor `name` as fp32 (BF16 widened exactly: bits << 16), n values.
int qe_safetensors_f32(const QeSafetensors* s, const char* name, float* out, int64_t n) {
    auto it = s->index.find(name);
    if (it == s->index.end() || !s->tensors[it->second].kept) {
        g_st_error = std::string("missing tensor: ") + name;
        return -1;
    }
    const Entry& e = s->tensors[it->second];
    const size_t count = e.dtype == QE_ST_BF16 ? e.bits.size() : e.values.size();
    if (n != int64_t(count)) {
        g_st_error = std::string("tensor shape mismatch: ") + name;
        return -1;
    }
    if (e.dtype == QE_ST_BF16) {
        for (size_t i = 0; i < count; ++i) {
            const uint32_t u = uint32_t(e.bits[i]) << 16;
            std::memcpy(out + i, &u, 4);
        }
    } else {
        std::memcpy(out, e.values.data(), count * 4);
    }
    return 0;
}

// BF16 bits of a BF16 tensor.
int qe_safetensors_bf16(const QeSafetensors* s, const char* name, uint16_t* out, int64_t n) {
    auto it = s->index.find(name);
    if (it == s->index.end() || !s->tensors[it->second].kept || s->tensors[it->second].dtype != QE_ST_BF16 ||
        int64_t(s->tensors[it->second].bits.size()) != n) {
        g_st_error = std::string("missing BF16 tensor or shape mismatch: ") + name;
        return -1;
    }
    std::memcpy(out, s->tensors[it->second].bits.data(), size_t(n) * 2);
    return 0;
}

}  // extern "C"
