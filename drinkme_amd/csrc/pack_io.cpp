// Pack tensor files without NumPy. One tensor of a drinkme pack is one
// .npz: a ZIP of stored .npy members, the arrays its codec names, plus
// `scalars`, a one-element unicode array holding the tensor's scalars as
// JSON (src/drinkme/codec/pack.py:509-520 writes it, :629-644 reads it).
//
// dmx_pack_read reads such a file through drinkme's load gates, in
// drinkme's words: the codec named by the scalars (pack.py:119-145), the
// shape and the allocation cap read off the ZIP directory before any array
// is touched (pack.py:164-207), then the descriptor gate (pack.py:210-276,
// radix.py:139-146 and :174-238). dmx_pack_write writes a file np.load
// reads back to the same arrays and the same scalars string.
//
// The file is memory-mapped; arrays are copied once, straight from the
// mapping into the caller's buffers (which may be pinned staging memory).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "dmx_radix.h"

namespace {

constexpr uint64_t kMaxTensorWeights = 1ull << 33;  // pack.py MAX_TENSOR_WEIGHTS
constexpr uint64_t kNpyHeaderSlack = 4096;           // pack.py _NPY_HEADER_SLACK
constexpr uint32_t kBlock = 1024;
constexpr uint32_t kMant = 7, kExp = 8;

int fail(char* err, size_t n, const std::string& msg) {
    if (err && n) {
        std::snprintf(err, n, "%s", msg.c_str());
    }
    return 1;
}

uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t rd64(const uint8_t* p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

// 1234567 -> "1,234,567" (Python's f"{n:,}")
std::string commas(uint64_t v) {
    std::string s = std::to_string(v), out;
    for (size_t i = 0; i < s.size(); ++i) {
        if (i && (s.size() - i) % 3 == 0) out += ',';
        out += s[i];
    }
    return out;
}

// ------------------------------------------------------------ the mapping --

struct Mapped {
    const uint8_t* p = nullptr;
    uint64_t n = 0;
    Mapped() = default;
    Mapped(const Mapped&) = delete;
    Mapped& operator=(const Mapped&) = delete;
    ~Mapped() {
        if (p) munmap(const_cast<uint8_t*>(p), n);
    }
    bool open(const char* path, std::string& err) {
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) {
            err = std::string(path) + ": " + std::strerror(errno);
            return false;
        }
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) {
            err = std::string(path) + ": empty or unreadable file";
            ::close(fd);
            return false;
        }
        void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        ::close(fd);
        if (m == MAP_FAILED) {
            err = std::string(path) + ": mmap: " + std::strerror(errno);
            return false;
        }
        p = static_cast<const uint8_t*>(m);
        n = (uint64_t)st.st_size;
        return true;
    }
    bool has(uint64_t off, uint64_t len) const { return off <= n && len <= n - off; }
};

// ---------------------------------------------------------------- the zip --

struct Member {
    std::string name;
    uint16_t method = 0, flags = 0;
    uint64_t csize = 0, usize = 0, local = 0;
};

// The central directory (ZIP64 records where the sizes call for them).
bool zip_members(const Mapped& f, std::vector<Member>& out, std::string& err) {
    const std::string bad = "not a ZIP archive (an .npz)";
    if (f.n < 22) {
        err = bad;
        return false;
    }
    uint64_t eocd = UINT64_MAX;
    const uint64_t lowest = f.n > 22 + 65535 ? f.n - 22 - 65535 : 0;
    for (uint64_t at = f.n - 22 + 1; at-- > lowest;) {
        if (rd32(f.p + at) == 0x06054b50u) {
            eocd = at;
            break;
        }
    }
    if (eocd == UINT64_MAX) {
        err = bad;
        return false;
    }
    uint64_t entries = rd16(f.p + eocd + 10), cd_size = rd32(f.p + eocd + 12), cd_off = rd32(f.p + eocd + 16);
    if (entries == 0xFFFF || cd_size == 0xFFFFFFFFu || cd_off == 0xFFFFFFFFu) {
        if (eocd < 20 || rd32(f.p + eocd - 20) != 0x07064b50u) {
            err = "ZIP64 end record missing";
            return false;
        }
        const uint64_t z = rd64(f.p + eocd - 20 + 8);
        if (!f.has(z, 56) || rd32(f.p + z) != 0x06064b50u) {
            err = "ZIP64 end record missing";
            return false;
        }
        entries = rd64(f.p + z + 32);
        cd_size = rd64(f.p + z + 40);
        cd_off = rd64(f.p + z + 48);
    }
    if (!f.has(cd_off, cd_size)) {
        err = "ZIP central directory out of the file";
        return false;
    }
    uint64_t at = cd_off;
    for (uint64_t e = 0; e < entries; ++e) {
        if (!f.has(at, 46) || rd32(f.p + at) != 0x02014b50u) {
            err = "ZIP central directory entry malformed";
            return false;
        }
        Member m;
        m.flags = rd16(f.p + at + 8);
        m.method = rd16(f.p + at + 10);
        m.csize = rd32(f.p + at + 20);
        m.usize = rd32(f.p + at + 24);
        const uint16_t nlen = rd16(f.p + at + 28), xlen = rd16(f.p + at + 30), clen = rd16(f.p + at + 32);
        m.local = rd32(f.p + at + 42);
        if (!f.has(at + 46, (uint64_t)nlen + xlen + clen)) {
            err = "ZIP central directory entry malformed";
            return false;
        }
        m.name.assign(reinterpret_cast<const char*>(f.p + at + 46), nlen);
        // ZIP64 extra: the 64-bit values, in order, of the fields set to all ones
        for (uint64_t x = at + 46 + nlen, end = x + xlen; x + 4 <= end;) {
            const uint16_t id = rd16(f.p + x), sz = rd16(f.p + x + 2);
            if (x + 4 + sz > end) break;
            if (id == 1) {
                uint64_t q = x + 4;
                const uint64_t qend = q + sz;
                if (m.usize == 0xFFFFFFFFu && q + 8 <= qend) m.usize = rd64(f.p + q), q += 8;
                if (m.csize == 0xFFFFFFFFu && q + 8 <= qend) m.csize = rd64(f.p + q), q += 8;
                if (m.local == 0xFFFFFFFFu && q + 8 <= qend) m.local = rd64(f.p + q), q += 8;
            }
            x += 4 + sz;
        }
        out.push_back(std::move(m));
        at += 46 + (uint64_t)nlen + xlen + clen;
    }
    return true;
}

// A member's stored bytes.
bool member_bytes(const Mapped& f, const Member& m, const uint8_t** data, std::string& err) {
    if (m.flags & 1u) {
        err = m.name + ": encrypted ZIP member";
        return false;
    }
    if (m.method != 0) {
        err = m.name + ": compressed ZIP member (method " + std::to_string(m.method) +
              "); pack tensors are written stored, as numpy.savez writes them";
        return false;
    }
    if (m.csize != m.usize || !f.has(m.local, 30) || rd32(f.p + m.local) != 0x04034b50u) {
        err = m.name + ": ZIP local header malformed";
        return false;
    }
    const uint64_t start = m.local + 30 + rd16(f.p + m.local + 26) + rd16(f.p + m.local + 28);
    if (!f.has(start, m.csize)) {
        err = m.name + ": ZIP member runs past the end of the file";
        return false;
    }
    *data = f.p + start;
    return true;
}

// ---------------------------------------------------------------- the npy --

struct Npy {
    std::string descr;  // as written: '<u4', '|u1', '<U64', ...
    bool fortran = false;
    std::vector<uint64_t> shape;
    const uint8_t* data = nullptr;
    uint64_t nbytes = 0;
    uint64_t count() const {
        uint64_t c = 1;
        for (uint64_t d : shape) c *= d;
        return c;
    }
};

// The item size of a descr (0 for one this reader does not size).
uint64_t item_size(const std::string& d) {
    if (d.size() < 3) return 0;
    const char kind = d[1];
    const uint64_t n = std::strtoull(d.c_str() + 2, nullptr, 10);
    if (kind == 'U') return 4 * n;
    if (kind == 'u' || kind == 'i' || kind == 'f' || kind == 'b') return n;
    return 0;
}

// NumPy's name of a descr (for the gates' messages).
std::string dtype_name(const std::string& d) {
    if (d.size() < 3) return d;
    const std::string bits = std::to_string(8 * std::strtoull(d.c_str() + 2, nullptr, 10));
    switch (d[1]) {
        case 'u': return "uint" + bits;
        case 'i': return "int" + bits;
        case 'f': return "float" + bits;
        case 'b': return "bool";
        default: return d;
    }
}

bool parse_npy(const uint8_t* p, uint64_t n, Npy& out, std::string& err) {
    if (n < 10 || std::memcmp(p, "\x93NUMPY", 6) != 0) {
        err = "not a .npy array";
        return false;
    }
    const uint8_t major = p[6];
    const uint64_t hstart = major == 1 ? 10 : 12;
    if (major < 1 || major > 3 || n < hstart) {
        err = ".npy version not understood";
        return false;
    }
    const uint64_t hlen = major == 1 ? rd16(p + 8) : rd32(p + 8);
    if (hstart + hlen > n) {
        err = ".npy header runs past the member";
        return false;
    }
    const std::string h(reinterpret_cast<const char*>(p + hstart), hlen);
    auto value_at = [&](const char* key) -> size_t {
        const size_t k = h.find(key);
        if (k == std::string::npos) return std::string::npos;
        const size_t c = h.find(':', k);
        return c == std::string::npos ? c : h.find_first_not_of(' ', c + 1);
    };
    size_t v = value_at("'descr'");
    if (v == std::string::npos || (h[v] != '\'' && h[v] != '"')) {
        err = ".npy header has no descr";
        return false;
    }
    const size_t e = h.find(h[v], v + 1);
    if (e == std::string::npos) {
        err = ".npy header has no descr";
        return false;
    }
    out.descr = h.substr(v + 1, e - v - 1);
    v = value_at("'fortran_order'");
    out.fortran = v != std::string::npos && h.compare(v, 4, "True") == 0;
    v = value_at("'shape'");
    if (v == std::string::npos || h[v] != '(') {
        err = ".npy header has no shape";
        return false;
    }
    const size_t close = h.find(')', v);
    if (close == std::string::npos) {
        err = ".npy header has no shape";
        return false;
    }
    out.shape.clear();
    for (size_t q = v + 1; q < close;) {
        q = h.find_first_not_of(" ,", q);
        if (q >= close) break;
        char* endp = nullptr;
        const unsigned long long d = std::strtoull(h.c_str() + q, &endp, 10);
        if (endp == h.c_str() + q) {
            err = ".npy shape not understood";
            return false;
        }
        out.shape.push_back(d);
        q = endp - h.c_str();
    }
    out.data = p + hstart + hlen;
    out.nbytes = n - hstart - hlen;
    const uint64_t isz = item_size(out.descr);
    if (isz == 0 || out.fortran || out.nbytes != out.count() * isz) {
        err = ".npy array of descr " + out.descr + " does not match its shape";
        return false;
    }
    return true;
}

// ---------------------------------------------------------------- the json --

struct JVal {
    enum Kind { Null, Bool, Int, Float, Str, Arr, Obj } kind = Null;
    bool b = false;
    int64_t i = 0;
    double d = 0;
    std::string s;  // Str; also the token text of a number
    std::vector<JVal> a;
    std::vector<std::pair<std::string, JVal>> o;
};

struct JParse {
    const std::string& t;
    size_t i = 0;
    explicit JParse(const std::string& s) : t(s) {}
    void ws() {
        while (i < t.size() && (t[i] == ' ' || t[i] == '\t' || t[i] == '\n' || t[i] == '\r')) ++i;
    }
    bool str(std::string& out) {
        if (i >= t.size() || t[i] != '"') return false;
        ++i;
        out.clear();
        while (i < t.size() && t[i] != '"') {
            char c = t[i++];
            if (c == '\\') {
                if (i >= t.size()) return false;
                const char esc = t[i++];
                switch (esc) {
                    case '"': c = '"'; break;
                    case '\\': c = '\\'; break;
                    case '/': c = '/'; break;
                    case 'b': c = '\b'; break;
                    case 'f': c = '\f'; break;
                    case 'n': c = '\n'; break;
                    case 'r': c = '\r'; break;
                    case 't': c = '\t'; break;
                    case 'u': {
                        if (i + 4 > t.size()) return false;
                        const unsigned cp = (unsigned)std::strtoul(t.substr(i, 4).c_str(), nullptr, 16);
                        i += 4;
                        if (cp < 0x80) {
                            c = (char)cp;
                        } else if (cp < 0x800) {
                            out += (char)(0xC0 | (cp >> 6));
                            c = (char)(0x80 | (cp & 0x3F));
                        } else {
                            out += (char)(0xE0 | (cp >> 12));
                            out += (char)(0x80 | ((cp >> 6) & 0x3F));
                            c = (char)(0x80 | (cp & 0x3F));
                        }
                        break;
                    }
                    default: return false;
                }
            }
            out += c;
        }
        if (i >= t.size()) return false;
        ++i;
        return true;
    }
    bool value(JVal& v, int depth = 0) {
        if (depth > 16) return false;
        ws();
        if (i >= t.size()) return false;
        const char c = t[i];
        if (c == '{') {
            v.kind = JVal::Obj;
            ++i;
            ws();
            if (i < t.size() && t[i] == '}') return ++i, true;
            for (;;) {
                ws();
                std::string k;
                if (!str(k)) return false;
                ws();
                if (i >= t.size() || t[i++] != ':') return false;
                JVal x;
                if (!value(x, depth + 1)) return false;
                v.o.emplace_back(std::move(k), std::move(x));
                ws();
                if (i < t.size() && t[i] == ',') {
                    ++i;
                    continue;
                }
                if (i < t.size() && t[i] == '}') return ++i, true;
                return false;
            }
        }
        if (c == '[') {
            v.kind = JVal::Arr;
            ++i;
            ws();
            if (i < t.size() && t[i] == ']') return ++i, true;
            for (;;) {
                JVal x;
                if (!value(x, depth + 1)) return false;
                v.a.push_back(std::move(x));
                ws();
                if (i < t.size() && t[i] == ',') {
                    ++i;
                    continue;
                }
                if (i < t.size() && t[i] == ']') return ++i, true;
                return false;
            }
        }
        if (c == '"') {
            v.kind = JVal::Str;
            return str(v.s);
        }
        if (t.compare(i, 4, "true") == 0) return v.kind = JVal::Bool, v.b = true, i += 4, true;
        if (t.compare(i, 5, "false") == 0) return v.kind = JVal::Bool, i += 5, true;
        if (t.compare(i, 4, "null") == 0) return v.kind = JVal::Null, i += 4, true;
        const size_t s0 = i;
        while (i < t.size() && std::strchr("+-0123456789.eE", t[i])) ++i;
        if (i == s0) return false;
        v.s = t.substr(s0, i - s0);
        if (v.s.find_first_of(".eE") == std::string::npos) {
            v.kind = JVal::Int;
            errno = 0;
            v.i = std::strtoll(v.s.c_str(), nullptr, 10);
            if (errno) v.kind = JVal::Float, v.d = std::strtod(v.s.c_str(), nullptr);
        } else {
            v.kind = JVal::Float;
            v.d = std::strtod(v.s.c_str(), nullptr);
        }
        return true;
    }
};

const JVal* jget(const JVal& obj, const char* key) {
    for (const auto& kv : obj.o)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

// Python's repr of a JSON scalar value (for the gates' messages).
std::string py_repr(const JVal* v) {
    if (!v) return "None";
    switch (v->kind) {
        case JVal::Null: return "None";
        case JVal::Bool: return v->b ? "True" : "False";
        case JVal::Int: return v->s;
        case JVal::Float: return v->s;
        case JVal::Str: return "'" + v->s + "'";
        case JVal::Arr: {
            std::string s = "[";
            for (size_t k = 0; k < v->a.size(); ++k) s += (k ? ", " : "") + py_repr(&v->a[k]);
            return s + "]";
        }
        default: return "{...}";
    }
}

// The shortest text that reads back as d, as Python's repr (and
// json.dumps) writes a float: 16.0, 11.219100952148438.
std::string float_text(double d) {
    if (std::isnan(d)) return "NaN";
    if (std::isinf(d)) return d > 0 ? "Infinity" : "-Infinity";
    char buf[40];
    for (int prec = 1; prec <= 17; ++prec) {
        std::snprintf(buf, sizeof buf, "%.*g", prec, d);
        if (std::strtod(buf, nullptr) == d) break;
    }
    std::string s = buf;
    if (s.find_first_of(".en") == std::string::npos) s += ".0";
    // C writes e+16 / e-05, as Python does; nothing else to change
    return s;
}

// ------------------------------------------------------------ the gates --

// block_word_bounds (radix.py:149-171): the fewest and the most words a
// block of n weights occupies.
void block_bounds(uint64_t n, const uint32_t* w, uint32_t nw, uint64_t& fewest, uint64_t& most) {
    auto per = [](uint64_t k, uint64_t width) { return (k * width + 31) / 32; };
    fewest = per(n, kMant + 1) + per(n, w[0]);
    most = fewest;
    for (uint32_t t = 1; t + 1 < nw; ++t) most += per(n, w[t]);
    most += per(n, kExp);
}

struct Tensor {
    std::string name, kind;  // kind: the codec scalar, "?" when absent
    JVal sc;
    uint64_t R = 0, C = 0;
    std::vector<Member> members;
};

std::string where(const Tensor& t) { return "pack tensor " + t.name + " (" + t.kind + "): "; }

const Member* find_member(const Tensor& t, const std::string& fn) {
    for (const auto& m : t.members)
        if (m.name == fn) return &m;
    return nullptr;
}

// The codec's arrays (pack.py:119-145), the shape (:164-171) and the
// allocation cap off the ZIP directory (:178-207).
int gate_directory(Tensor& t, std::vector<std::string>& arrays, std::string& err) {
    const JVal* codec = jget(t.sc, "codec");
    const JVal* dtype = jget(t.sc, "dtype");
    const std::string nm = t.name.empty() ? "<unnamed>" : t.name;
    if (codec && codec->kind == JVal::Str && codec->s == "radix") {
        arrays = {"rx_palette", "rx_offsets", "rx_data"};
    } else if (codec && codec->kind == JVal::Str && codec->s == "raw") {
        arrays = {"raw_bits"};
    } else if (codec && codec->kind != JVal::Null) {
        err = "pack tensor " + nm + " declares codec " + py_repr(codec) +
              ", which this build does not implement (knows 'radix' and 'raw') — refusing to load.";
        return 1;
    } else if (dtype && dtype->kind != JVal::Null) {
        err = "pack tensor " + nm + " (dtype " + py_repr(dtype) +
              "): a tensor kind this build does not serve; re-pack from a bf16 checkpoint";
        return 1;
    } else {
        err = "pack tensor " + nm +
              " names no codec ('radix' | 'raw') — not a pack format 1 tensor; refusing to load.";
        return 1;
    }
    t.kind = codec->s;
    const JVal *R = jget(t.sc, "R"), *C = jget(t.sc, "C");
    if (!R || !C || R->kind != JVal::Int || C->kind != JVal::Int || R->i <= 0 || C->i <= 0) {
        err = where(t) + "R, C must be positive ints, got " + py_repr(R) + ", " + py_repr(C);
        return 1;
    }
    t.R = (uint64_t)R->i;
    t.C = (uint64_t)C->i;
    if (t.R > kMaxTensorWeights || t.C > kMaxTensorWeights || t.R * t.C > kMaxTensorWeights) {
        err = where(t) + "R x C = " + commas(t.R) + " x " + commas(t.C) + " is " + commas(t.R * t.C) +
              " weights, more than the " + commas(kMaxTensorWeights) + " this loader will allocate for";
        return 1;
    }
    const uint64_t plane = 2 * t.R * t.C;
    for (const auto& key : arrays) {
        const Member* m = find_member(t, key + ".npy");
        if (!m) {
            std::vector<std::string> names;
            for (const auto& x : t.members) names.push_back(x.name);
            std::sort(names.begin(), names.end());
            std::string list = "[";
            for (size_t k = 0; k < names.size(); ++k) list += (k ? ", '" : "'") + names[k] + "'";
            err = where(t) + "declares R x C = " + std::to_string(t.R) + " x " + std::to_string(t.C) +
                  " but the npz holds no " + key + ".npy (members: " + list + "])";
            return 1;
        }
        if (m->usize > plane + kNpyHeaderSlack) {
            const std::string what = t.kind == "radix"
                                         ? "the 2 x R x C = " + commas(plane) + " the tensor's bf16 plane takes"
                                         : "the 2 x R x C = " + commas(plane) + " bytes of bf16 bits it declares";
            err = where(t) + key + ".npy is " + commas(m->usize) + " bytes, more than " + what +
                  " — refusing to allocate it";
            return 1;
        }
    }
    return 0;
}

// The served line and radix.validate (pack.py:210-276, radix.py:139-146,
// :174-238) on the arrays as read.
int gate_radix(const Tensor& t, const Npy& pal, const Npy& off, const Npy& dat, dmx_pack_info* info,
               std::string& err) {
    const JVal* W = jget(t.sc, "widths");
    bool ok = W && W->kind == JVal::Arr && W->a.size() >= 2;
    if (ok)
        for (const auto& x : W->a) ok = ok && x.kind == JVal::Int;
    if (!ok) {
        err = where(t) + "widths " + py_repr(W) + " is not a list of 2+ ints";
        return 1;
    }
    const std::string wl = py_repr(W);
    const JVal* B = jget(t.sc, "block_size");
    if (!B || B->kind != JVal::Int || B->i != (int64_t)kBlock) {
        err = where(t) + "block_size " + py_repr(B) + " — the served kernels walk 1024-weight blocks only";
        return 1;
    }
    const size_t nw = W->a.size();
    if (nw > 4) {
        err = where(t) + "widths " + wl + " is " + std::to_string(nw) +
              " tiers; the scheduled decoder's block header holds at most four (three nonterminal)";
        return 1;
    }
    for (size_t k = 0; k + 1 < nw; ++k)
        if (W->a[k].i < 1 || W->a[k].i > 4) {
            err = where(t) + "widths " + wl +
                  " — a nonterminal tier must be 1..4 bits (one byte of the block header per tier)";
            return 1;
        }
    if (W->a[nw - 1].i != 8) {
        err = where(t) + "widths " + wl + " — the terminal tier is the 8-bit bf16 exponent";
        return 1;
    }
    const JVal* P = jget(t.sc, "profile");
    if (!P || P->kind != JVal::Str || (P->s != "sip" && P->s != "balanced" && P->s != "gulp")) {
        err = where(t) + "profile " + py_repr(P) +
              " is not one this drinkme packs or serves (sip | gulp); re-pack with "
              "`drinkme pack --model <repo> --replace`";
        return 1;
    }
    uint32_t w[8];
    uint64_t covered = 0;
    for (size_t k = 0; k < nw; ++k) w[k] = (uint32_t)W->a[k].i;
    for (size_t k = 0; k + 1 < nw; ++k) covered += (1u << w[k]) - 1;
    const std::string pre = where(t);
    if (covered > 256) {
        err = pre + "radix tiers exceed the exponent alphabet";
        return 1;
    }
    if (pal.shape.size() != 1 || (pal.descr != "|u1" && pal.descr != "<u1")) {
        err = pre + "invalid radix palette";
        return 1;
    }
    if (off.shape.size() != 1 || off.descr != "<u4") {
        err = pre + "invalid radix directory";
        return 1;
    }
    const uint64_t per_row = (t.C + kBlock - 1) / kBlock, nb = t.R * per_row;
    {
        bool seen[256] = {};
        bool good = pal.count() == covered;
        for (uint64_t k = 0; good && k < covered; ++k) {
            good = !seen[pal.data[k]];
            seen[pal.data[k]] = true;
        }
        if (!good) {
            err = pre + "invalid radix palette entries";
            return 1;
        }
    }
    if (dat.shape.size() != 1 || dat.descr != "<u4") {
        err = pre + "invalid radix payload";
        return 1;
    }
    const uint8_t* o = off.data;
    const uint64_t n_off = off.count();
    if (n_off != nb + 1 || rd32(o) != 0 || rd32(o + 4 * nb) != dat.count()) {
        err = pre + "invalid radix block offsets";
        return 1;
    }
    for (uint64_t k = 0; k < nb; ++k)
        if (rd32(o + 4 * (k + 1)) <= rd32(o + 4 * k)) {
            err = pre + "invalid radix block offsets";
            return 1;
        }
    // the extents against the fixed streams, then the widest block
    for (int pass = 0; pass < 2; ++pass)
        for (uint64_t k = 0; k < nb; ++k) {
            const uint64_t n = std::min<uint64_t>(kBlock, t.C - (k % per_row) * kBlock);
            uint64_t fewest, most;
            block_bounds(n, w, (uint32_t)nw, fewest, most);
            const uint64_t len = (uint64_t)rd32(o + 4 * (k + 1)) - rd32(o + 4 * k);
            if (pass == 0 && len < fewest) {
                err = pre + "invalid radix block offsets: block " + std::to_string(k) + " holds " +
                      std::to_string(len) + " word(s), fewer than the " + std::to_string(fewest) +
                      " its literal plane and first tier take for " + std::to_string(n) + " weights";
                return 1;
            }
            if (pass == 1 && len > most) {
                err = pre + "invalid radix block offsets: block " + std::to_string(k) + " holds " +
                      std::to_string(len) + " words, more than the " + std::to_string(most) + " any block of " +
                      std::to_string(n) + " weights can use";
                return 1;
            }
        }
    if (info) {
        info->n_widths = (uint32_t)nw;
        for (size_t k = 0; k < 8; ++k) info->widths[k] = k < nw ? w[k] : 0;
        std::snprintf(info->profile, sizeof info->profile, "%s", P->s.c_str());
        info->block_size = kBlock;
    }
    return 0;
}

int gate_raw(const Tensor& t, const Npy& bits, std::string& err) {
    if (bits.descr != "<u2") {
        err = where(t) + "raw_bits dtype " + dtype_name(bits.descr) + ", not uint16";
        return 1;
    }
    if (bits.shape.size() != 2 || bits.shape[0] != t.R || bits.shape[1] != t.C) {
        std::string s = "(";
        for (size_t k = 0; k < bits.shape.size(); ++k) s += (k ? ", " : "") + std::to_string(bits.shape[k]);
        s += bits.shape.size() == 1 ? ",)" : ")";
        err = where(t) + "raw_bits is " + s + ", not [R, C] = (" + std::to_string(t.R) + ", " + std::to_string(t.C) +
              ")";
        return 1;
    }
    return 0;
}

// The scalars member: a one-element unicode array holding JSON.
int read_scalars(const Mapped& f, Tensor& t, std::string& err) {
    const Member* m = find_member(t, "scalars.npy");
    if (!m) {
        err = "pack tensor " + t.name + ": the npz holds no scalars.npy";
        return 1;
    }
    const uint8_t* p = nullptr;
    Npy a;
    if (!member_bytes(f, *m, &p, err) || !parse_npy(p, m->usize, a, err)) {
        err = "pack tensor " + t.name + ": scalars: " + err;
        return 1;
    }
    if (a.descr.size() < 3 || a.descr[1] != 'U' || a.count() != 1) {
        err = "pack tensor " + t.name + ": scalars is not a one-element unicode array";
        return 1;
    }
    std::string s;
    const uint64_t chars = a.nbytes / 4;
    for (uint64_t k = 0; k < chars; ++k) {
        const uint32_t cp = a.descr[0] == '>' ? __builtin_bswap32(rd32(a.data + 4 * k)) : rd32(a.data + 4 * k);
        if (cp == 0) break;
        if (cp < 0x80) {
            s += (char)cp;
        } else if (cp < 0x800) {
            s += (char)(0xC0 | (cp >> 6));
            s += (char)(0x80 | (cp & 0x3F));
        } else if (cp < 0x10000) {
            s += (char)(0xE0 | (cp >> 12));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        } else {
            s += (char)(0xF0 | (cp >> 18));
            s += (char)(0x80 | ((cp >> 12) & 0x3F));
            s += (char)(0x80 | ((cp >> 6) & 0x3F));
            s += (char)(0x80 | (cp & 0x3F));
        }
    }
    JParse jp(s);
    if (!jp.value(t.sc) || t.sc.kind != JVal::Obj) {
        err = "pack tensor " + t.name + ": scalars is not a JSON object";
        return 1;
    }
    return 0;
}

// ------------------------------------------------------------ the writer --

uint32_t crc32_update(uint32_t crc, const uint8_t* p, uint64_t n) {
    static uint32_t table[256];
    static bool ready = false;
    if (!ready) {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
            table[i] = c;
        }
        ready = true;
    }
    crc = ~crc;
    for (uint64_t i = 0; i < n; ++i) crc = table[(crc ^ p[i]) & 0xFF] ^ (crc >> 8);
    return ~crc;
}

// A .npy v1.0 header for a little-endian C-order array, padded (as NumPy
// pads it) so the data starts on a 64-byte boundary.
std::string npy_header(const std::string& descr, const std::vector<uint64_t>& shape) {
    std::string sh = "(";
    for (size_t k = 0; k < shape.size(); ++k) sh += (k ? ", " : "") + std::to_string(shape[k]);
    if (shape.size() == 1) sh += ",";
    sh += ")";
    std::string d = "{'descr': '" + descr + "', 'fortran_order': False, 'shape': " + sh + ", }";
    const size_t total = 10 + d.size() + 1;
    d.append((64 - total % 64) % 64, ' ');
    d += '\n';
    std::string h = "\x93NUMPY";
    h += '\x01';
    h += '\x00';
    h += (char)(d.size() & 0xFF);
    h += (char)(d.size() >> 8);
    return h + d;
}

struct Out {
    FILE* f = nullptr;
    uint64_t at = 0;
    bool ok = true;
    void put(const void* p, uint64_t n) {
        if (ok && n && std::fwrite(p, 1, n, f) != n) ok = false;
        at += n;
    }
    void u16(uint16_t v) {
        const uint8_t b[2] = {(uint8_t)v, (uint8_t)(v >> 8)};
        put(b, 2);
    }
    void u32(uint32_t v) {
        const uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
        put(b, 4);
    }
    void u64(uint64_t v) {
        u32((uint32_t)v);
        u32((uint32_t)(v >> 32));
    }
};

struct Written {
    std::string name;
    uint32_t crc;
    uint64_t size, local;
};

// One stored member: local header, the .npy header, the array bytes.
void write_member(Out& o, std::vector<Written>& dir, const std::string& name, const std::string& header,
                  const void* data, uint64_t nbytes) {
    const uint64_t size = header.size() + nbytes;
    uint32_t crc = crc32_update(0, reinterpret_cast<const uint8_t*>(header.data()), header.size());
    crc = crc32_update(crc, static_cast<const uint8_t*>(data), nbytes);
    const bool z64 = size >= 0xFFFFFFFFull;
    dir.push_back({name, crc, size, o.at});
    o.u32(0x04034b50u);
    o.u16(z64 ? 45 : 20);
    o.u16(0);  // flags
    o.u16(0);  // stored
    o.u16(0);  // time
    o.u16((1 << 5) | 1);  // 1980-01-01
    o.u32(crc);
    o.u32(z64 ? 0xFFFFFFFFu : (uint32_t)size);
    o.u32(z64 ? 0xFFFFFFFFu : (uint32_t)size);
    o.u16((uint16_t)name.size());
    o.u16(z64 ? 20 : 0);
    o.put(name.data(), name.size());
    if (z64) {
        o.u16(1);
        o.u16(16);
        o.u64(size);
        o.u64(size);
    }
    o.put(header.data(), header.size());
    o.put(data, nbytes);
}

void write_directory(Out& o, const std::vector<Written>& dir) {
    const uint64_t cd_off = o.at;
    for (const auto& w : dir) {
        const bool zs = w.size >= 0xFFFFFFFFull, zo = w.local >= 0xFFFFFFFFull;
        const uint16_t xlen = (uint16_t)((zs ? 16 : 0) + (zo ? 8 : 0));
        o.u32(0x02014b50u);
        o.u16(45);
        o.u16(xlen ? 45 : 20);
        o.u16(0);
        o.u16(0);
        o.u16(0);
        o.u16((1 << 5) | 1);
        o.u32(w.crc);
        o.u32(zs ? 0xFFFFFFFFu : (uint32_t)w.size);
        o.u32(zs ? 0xFFFFFFFFu : (uint32_t)w.size);
        o.u16((uint16_t)w.name.size());
        o.u16(xlen ? (uint16_t)(4 + xlen) : 0);
        o.u16(0);
        o.u16(0);
        o.u16(0);
        o.u32(0x01800000u);  // -rw------- as Python's zipfile records it
        o.u32(zo ? 0xFFFFFFFFu : (uint32_t)w.local);
        o.put(w.name.data(), w.name.size());
        if (xlen) {
            o.u16(1);
            o.u16(xlen);
            if (zs) {
                o.u64(w.size);
                o.u64(w.size);
            }
            if (zo) o.u64(w.local);
        }
    }
    const uint64_t cd_size = o.at - cd_off, n = dir.size();
    if (n >= 0xFFFF || cd_size >= 0xFFFFFFFFull || cd_off >= 0xFFFFFFFFull) {
        const uint64_t z = o.at;
        o.u32(0x06064b50u);
        o.u64(44);
        o.u16(45);
        o.u16(45);
        o.u32(0);
        o.u32(0);
        o.u64(n);
        o.u64(n);
        o.u64(cd_size);
        o.u64(cd_off);
        o.u32(0x07064b50u);
        o.u32(0);
        o.u64(z);
        o.u32(1);
    }
    o.u32(0x06054b50u);
    o.u16(0);
    o.u16(0);
    o.u16((uint16_t)std::min<uint64_t>(n, 0xFFFF));
    o.u16((uint16_t)std::min<uint64_t>(n, 0xFFFF));
    o.u32((uint32_t)std::min<uint64_t>(cd_size, 0xFFFFFFFFull));
    o.u32((uint32_t)std::min<uint64_t>(cd_off, 0xFFFFFFFFull));
    o.u16(0);
}

}  // namespace

extern "C" int dmx_pack_read(const char* path, const char* name, dmx_pack_info* info, uint8_t* palette,
                             uint32_t* offsets, uint32_t* data, uint16_t* raw_bits, char* err, size_t errn) {
    if (!path || !info) return fail(err, errn, "null path or info");
    std::string e;
    Mapped f;
    if (!f.open(path, e)) return fail(err, errn, e);
    Tensor t;
    t.name = name ? name : "";
    if (!zip_members(f, t.members, e)) return fail(err, errn, std::string(path) + ": " + e);
    if (read_scalars(f, t, e)) return fail(err, errn, e);
    std::vector<std::string> arrays;
    if (gate_directory(t, arrays, e)) return fail(err, errn, e);
    std::vector<Npy> npy(arrays.size());
    for (size_t k = 0; k < arrays.size(); ++k) {
        const Member* m = find_member(t, arrays[k] + ".npy");
        const uint8_t* p = nullptr;
        if (!member_bytes(f, *m, &p, e) || !parse_npy(p, m->usize, npy[k], e))
            return fail(err, errn, where(t) + arrays[k] + ": " + e);
    }
    std::memset(info, 0, sizeof *info);
    info->rows = t.R;
    info->cols = t.C;
    const JVal* bpw = jget(t.sc, "bpw");
    info->bpw = bpw && (bpw->kind == JVal::Float || bpw->kind == JVal::Int) ? (bpw->kind == JVal::Int ? (double)bpw->i : bpw->d)
                                                                             : NAN;
    if (t.kind == "radix") {
        info->codec = DMX_CODEC_RADIX;
        if (gate_radix(t, npy[0], npy[1], npy[2], info, e)) return fail(err, errn, e);
        info->palette_len = npy[0].count();
        info->offsets_len = npy[1].count();
        info->data_len = npy[2].count();
        if (palette) std::memcpy(palette, npy[0].data, npy[0].nbytes);
        if (offsets) std::memcpy(offsets, npy[1].data, npy[1].nbytes);
        if (data) std::memcpy(data, npy[2].data, npy[2].nbytes);
    } else {
        info->codec = DMX_CODEC_RAW;
        if (gate_raw(t, npy[0], e)) return fail(err, errn, e);
        if (raw_bits) std::memcpy(raw_bits, npy[0].data, npy[0].nbytes);
    }
    return 0;
}

extern "C" int dmx_pack_write(const char* path, const dmx_pack_info* info, const uint8_t* palette,
                              const uint32_t* offsets, const uint32_t* data, const uint16_t* raw_bits, char* err,
                              size_t errn) {
    if (!path || !info) return fail(err, errn, "null path or info");
    if (info->rows == 0 || info->cols == 0) return fail(err, errn, "empty tensor");
    std::string js;
    struct Arr {
        const char* name;
        std::string descr;
        std::vector<uint64_t> shape;
        const void* p;
        uint64_t nbytes;
    };
    std::vector<Arr> arrs;
    const std::string R = std::to_string(info->rows), C = std::to_string(info->cols);
    if (info->codec == DMX_CODEC_RADIX) {
        if (!palette || !offsets || !data) return fail(err, errn, "a radix tensor needs palette, offsets and data");
        if (info->n_widths < 2 || info->n_widths > 8) return fail(err, errn, "radix needs 2..8 widths");
        std::string wl = "[";
        for (uint32_t k = 0; k < info->n_widths; ++k) wl += (k ? ", " : "") + std::to_string(info->widths[k]);
        wl += "]";
        char prof[sizeof info->profile + 1] = {};
        std::memcpy(prof, info->profile, sizeof info->profile);
        // json.dumps of {k: pack[k] for k in _SCALARS_RADIX} (radix_pack.py:71)
        js = "{\"R\": " + R + ", \"C\": " + C + ", \"bpw\": " + float_text(info->bpw) +
             ", \"codec\": \"radix\", \"profile\": \"" + prof + "\", \"widths\": " + wl +
             ", \"block_size\": " + std::to_string(info->block_size) + "}";
        arrs.push_back({"rx_palette", "|u1", {info->palette_len}, palette, info->palette_len});
        arrs.push_back({"rx_offsets", "<u4", {info->offsets_len}, offsets, 4 * info->offsets_len});
        arrs.push_back({"rx_data", "<u4", {info->data_len}, data, 4 * info->data_len});
    } else if (info->codec == DMX_CODEC_RAW) {
        if (!raw_bits) return fail(err, errn, "a raw tensor needs raw_bits");
        js = "{\"R\": " + R + ", \"C\": " + C + ", \"bpw\": " + float_text(info->bpw) + ", \"codec\": \"raw\"}";
        arrs.push_back({"raw_bits", "<u2", {info->rows, info->cols}, raw_bits, 2 * info->rows * info->cols});
    } else {
        return fail(err, errn, "codec must be DMX_CODEC_RADIX or DMX_CODEC_RAW");
    }
    std::vector<uint8_t> sc(4 * js.size());
    for (size_t k = 0; k < js.size(); ++k) sc[4 * k] = (uint8_t)js[k];
    const std::string tmp = std::string(path) + ".tmp";
    Out o;
    o.f = std::fopen(tmp.c_str(), "wb");
    if (!o.f) return fail(err, errn, tmp + ": " + std::strerror(errno));
    std::vector<Written> dir;
    for (const auto& a : arrs) write_member(o, dir, std::string(a.name) + ".npy", npy_header(a.descr, a.shape), a.p, a.nbytes);
    write_member(o, dir, "scalars.npy", npy_header("<U" + std::to_string(js.size()), {1}), sc.data(), sc.size());
    write_directory(o, dir);
    const bool closed = std::fclose(o.f) == 0;
    if (!o.ok || !closed) {
        std::remove(tmp.c_str());
        return fail(err, errn, tmp + ": write failed");
    }
    if (std::rename(tmp.c_str(), path) != 0) {
        std::remove(tmp.c_str());
        return fail(err, errn, std::string(path) + ": " + std::strerror(errno));
    }
    return 0;
}
