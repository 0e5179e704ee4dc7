// Host half of libdmx_radix.so: the radix codec on CPU threads, and the
// seeded synthetic generator.
//
// dmx_radix_native stands in for drinkme's radix_native
// (src/drinkme/codec/radix_native.cpp:211-236): the same ops, arguments,
// results and refusal messages, so drinkme's ctypes wrapper
// (src/drinkme/codec/radix_native.py:166-184) can bind it unchanged. The
// byte layout it writes is the format's (radix.py:77-136); the code here is
// organised for threads: the directory is a prefix sum over independent
// per-block sizes, and every block is then encoded or decoded on its own
// with a streaming bit writer / reader.
#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "dmx_radix.h"

namespace {

std::atomic<int> g_threads{0};

int resolve_threads() {
    int n = g_threads.load();
    if (n <= 0) {
        unsigned hc = std::thread::hardware_concurrency();
        n = hc ? static_cast<int>(hc) : 1;
    }
    return std::min(n, 16);
}

// Runs fn(begin, end) over [0, count) split into contiguous chunks, one
// per thread; the first exception is rethrown on the caller's thread.
template <class Fn>
void parallel_for(uint64_t count, uint64_t min_chunk, Fn fn) {
    int threads = resolve_threads();
    uint64_t chunks = std::min<uint64_t>(threads, (count + min_chunk - 1) / std::max<uint64_t>(min_chunk, 1));
    if (chunks <= 1) {
        fn(uint64_t(0), count);
        return;
    }
    std::vector<std::thread> pool;
    std::vector<std::string> errors(chunks);
    for (uint64_t t = 0; t < chunks; ++t) {
        uint64_t b = count * t / chunks, e = count * (t + 1) / chunks;
        pool.emplace_back([&, b, e, t] {
            try {
                fn(b, e);
            } catch (const std::exception& ex) {
                errors[t] = ex.what();
            }
        });
    }
    for (auto& th : pool) th.join();
    for (auto& e : errors)
        if (!e.empty()) throw std::runtime_error(e);
}

constexpr uint64_t kBlock = 1024;

uint64_t stream_words(uint64_t count, uint32_t width) { return (count * width + 31) / 32; }

// The tensor's geometry and code tables: tier j covers palette ranks
// [first[j], first[j] + (1 << w_j) - 1); the padded device table of tier j
// starts at byte table[j] of a region's `stride` bytes.
struct Geometry {
    uint64_t rows, cols, rg, cg, nb, regions_per_col, regions;
    uint32_t mant, exponent, tiers, covered, stride;
    uint32_t width[8], first[8], table[8];

    Geometry(uint64_t r, uint64_t c, uint64_t row_group, uint64_t block_group, uint32_t m, uint32_t e,
             const uint32_t* w, uint32_t nw)
        : rows(r), cols(c), rg(row_group), cg(block_group), mant(m), exponent(e), tiers(nw) {
        if (!r || !c || !rg || !cg || r > (1ULL << 32) || c > (1ULL << 24) || !w ||
            !((m == 7 && e == 8) || (m == 3 && e == 4)) || nw < 2 || nw > 8 || w[nw - 1] != e)
            throw std::runtime_error("invalid layout");
        nb = (c + kBlock - 1) / kBlock;
        regions_per_col = (nb + cg - 1) / cg;
        regions = ((r + rg - 1) / rg) * regions_per_col;
        covered = stride = 0;
        for (uint32_t j = 0; j + 1 < nw; ++j) {
            if (w[j] < 1 || w[j] > 8) throw std::runtime_error("invalid width");
            width[j] = w[j];
            first[j] = covered;
            table[j] = stride;
            covered += (1u << w[j]) - 1;
            stride += (((1u << w[j]) + 2) / 4) * 4;
        }
        width[nw - 1] = e;
        if (covered > (1u << e)) throw std::runtime_error("palette exceeds alphabet");
    }
    uint64_t region(uint64_t row, uint64_t block) const { return (row / rg) * regions_per_col + block / cg; }
    uint64_t block_len(uint64_t block) const { return std::min(kBlock, cols - block * kBlock); }
};

// rank_of[region][exponent]: the palette rank, or `covered` when absent.
std::vector<uint16_t> rank_tables(const Geometry& g, const uint8_t* tables) {
    const uint32_t alphabet = 1u << g.exponent;
    std::vector<uint16_t> rank(g.regions * alphabet, static_cast<uint16_t>(g.covered));
    for (uint64_t reg = 0; reg < g.regions; ++reg) {
        const uint8_t* t = tables + reg * g.stride;
        uint16_t* rk = rank.data() + reg * alphabet;
        for (uint32_t j = 0; j + 1 < g.tiers; ++j) {
            uint32_t n = (1u << g.width[j]) - 1, padded = ((n + 3) / 4) * 4;
            for (uint32_t k = 0; k < n; ++k) {
                uint32_t e = t[g.table[j] + k];
                if (e >= alphabet || rk[e] != g.covered) throw std::runtime_error("invalid or repeated palette value");
                rk[e] = static_cast<uint16_t>(g.first[j] + k);
            }
            for (uint32_t k = n; k < padded; ++k)
                if (t[g.table[j] + k]) throw std::runtime_error("nonzero palette padding");
        }
    }
    return rank;
}

// Little-endian w-bit fields appended to a word stream.
struct BitWriter {
    uint32_t* out;
    uint64_t acc = 0;
    uint32_t bits = 0;
    explicit BitWriter(uint32_t* o) : out(o) {}
    void put(uint32_t v, uint32_t w) {
        acc |= static_cast<uint64_t>(v) << bits;
        bits += w;
        if (bits >= 32) {
            *out++ = static_cast<uint32_t>(acc);
            acc >>= 32;
            bits -= 32;
        }
    }
    uint32_t* finish() {
        if (bits) *out++ = static_cast<uint32_t>(acc);
        acc = 0;
        bits = 0;
        return out;
    }
};

struct BitReader {
    const uint32_t* in;
    uint64_t acc = 0;
    uint32_t bits = 0;
    explicit BitReader(const uint32_t* i) : in(i) {}
    uint32_t get(uint32_t w) {
        if (bits < w) {
            acc |= static_cast<uint64_t>(*in++) << bits;
            bits += 32;
        }
        uint32_t v = static_cast<uint32_t>(acc) & ((1u << w) - 1);
        acc >>= w;
        bits -= w;
        return v;
    }
};

template <class T>
uint32_t exponent_of(T v, const Geometry& g) {
    return (static_cast<uint32_t>(v) >> g.mant) & ((1u << g.exponent) - 1);
}

// op 0: histogram per region -> palette tables (count descending, ties by
// exponent ascending) -> per-block word counts -> directory.
template <class T>
uint64_t plan(const T* src, const Geometry& g, uint8_t* tables, uint32_t* offsets) {
    const uint32_t alphabet = 1u << g.exponent;
    const uint64_t row_groups = (g.rows + g.rg - 1) / g.rg;
    std::vector<uint64_t> hist(g.regions * alphabet, 0);
    auto count_rows = [&](uint64_t r0, uint64_t r1, uint64_t* into) {
        for (uint64_t row = r0; row < r1; ++row)
            for (uint64_t blk = 0; blk < g.nb; ++blk) {
                uint64_t* h = into + g.region(row, blk) * alphabet;
                const T* s = src + row * g.cols + blk * kBlock;
                for (uint64_t i = 0, n = g.block_len(blk); i < n; ++i) ++h[exponent_of(s[i], g)];
            }
    };
    if (g.regions <= 64) {
        // few regions (drinkme packs one per tensor): every thread counts a
        // row range into its own histograms, merged in thread order
        std::vector<std::vector<uint64_t>> part;
        std::mutex lock;
        parallel_for(g.rows, 64, [&](uint64_t b, uint64_t e) {
            std::vector<uint64_t> local(g.regions * alphabet, 0);
            count_rows(b, e, local.data());
            std::lock_guard<std::mutex> hold(lock);
            part.push_back(std::move(local));
        });
        for (const auto& p : part)
            for (size_t i = 0; i < hist.size(); ++i) hist[i] += p[i];
    } else {
        // many regions: one row group per thread owns its regions' counts
        parallel_for(row_groups, 1, [&](uint64_t b, uint64_t e) {
            for (uint64_t grp = b; grp < e; ++grp)
                count_rows(grp * g.rg, std::min(g.rows, (grp + 1) * g.rg), hist.data());
        });
    }
    std::memset(tables, 0, g.regions * g.stride);
    for (uint64_t reg = 0; reg < g.regions; ++reg) {
        const uint64_t* h = hist.data() + reg * alphabet;
        std::array<uint16_t, 256> order{};
        for (uint32_t e = 0; e < alphabet; ++e) order[e] = static_cast<uint16_t>(e);
        std::stable_sort(order.begin(), order.begin() + alphabet, [h](uint16_t a, uint16_t b) { return h[a] > h[b]; });
        for (uint32_t j = 0; j + 1 < g.tiers; ++j)
            for (uint32_t k = 0; k < (1u << g.width[j]) - 1; ++k)
                tables[reg * g.stride + g.table[j] + k] = static_cast<uint8_t>(order[g.first[j] + k]);
    }
    const auto rank = rank_tables(g, tables);
    const uint64_t nblocks = g.rows * g.nb;
    std::vector<uint64_t> words(nblocks);
    parallel_for(nblocks, 256, [&](uint64_t b, uint64_t e) {
        for (uint64_t id = b; id < e; ++id) {
            uint64_t row = id / g.nb, blk = id % g.nb, n = g.block_len(blk);
            const uint16_t* rk = rank.data() + g.region(row, blk) * alphabet;
            // escapes past tier j = weights whose rank is at least the
            // tier's last code
            std::array<uint32_t, 257> by_rank{};
            const T* s = src + row * g.cols + blk * kBlock;
            for (uint64_t i = 0; i < n; ++i) ++by_rank[rk[exponent_of(s[i], g)]];
            uint64_t total = stream_words(n, g.mant + 1), active = n;
            for (uint32_t j = 0; j + 1 < g.tiers; ++j) {
                total += stream_words(active, g.width[j]);
                for (uint32_t r = g.first[j]; r < g.first[j] + (1u << g.width[j]) - 1; ++r) active -= by_rank[r];
            }
            words[id] = total + stream_words(active, g.exponent);
        }
    });
    uint64_t sum = 0;
    offsets[0] = 0;
    for (uint64_t id = 0; id < nblocks; ++id) {
        sum += words[id];
        if (sum > UINT32_MAX) throw std::runtime_error("word directory overflow");
        offsets[id + 1] = static_cast<uint32_t>(sum);
    }
    return sum;
}

// op 1: every block written on its own, at the directory's offset.
template <class T>
void encode(const T* src, const Geometry& g, const uint8_t* tables, const uint32_t* offsets, uint32_t* data,
            uint64_t words) {
    const uint64_t nblocks = g.rows * g.nb;
    if (offsets[0] || offsets[nblocks] != words) throw std::runtime_error("directory endpoints");
    const uint32_t alphabet = 1u << g.exponent;
    const auto rank = rank_tables(g, tables);
    parallel_for(nblocks, 256, [&](uint64_t b, uint64_t e) {
        std::array<uint16_t, kBlock> rk_of, ex_of;
        for (uint64_t id = b; id < e; ++id) {
            uint64_t row = id / g.nb, blk = id % g.nb, n = g.block_len(blk);
            uint64_t pos = offsets[id], end = offsets[id + 1];
            if (end <= pos || end > words) throw std::runtime_error("invalid block bounds");
            const T* s = src + row * g.cols + blk * kBlock;
            const uint16_t* rk = rank.data() + g.region(row, blk) * alphabet;
            uint32_t* w = data + pos;
            uint32_t* stop = data + end;
            if (stream_words(n, g.mant + 1) > end - pos) throw std::runtime_error("short literal stream");
            BitWriter lit(w);
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t v = static_cast<uint32_t>(s[i]);
                lit.put((v & ((1u << g.mant) - 1)) | ((v >> (g.mant + g.exponent)) << g.mant), g.mant + 1);
                ex_of[i] = static_cast<uint16_t>(exponent_of(s[i], g));
                rk_of[i] = rk[ex_of[i]];
            }
            w = lit.finish();
            // tier j's stream: one code per weight still active, in order;
            // a weight stays active while its rank is past the tier's codes
            uint64_t active = n;
            for (uint32_t j = 0; j + 1 < g.tiers; ++j) {
                const uint32_t width = g.width[j], esc = (1u << width) - 1, base = g.first[j];
                if (static_cast<uint64_t>(stop - w) < stream_words(active, width))
                    throw std::runtime_error("short exponent stream");
                BitWriter tier(w);
                uint64_t kept = 0;
                for (uint64_t i = 0; i < active; ++i) {
                    uint32_t code = std::min<uint32_t>(rk_of[i] - base, esc);
                    tier.put(code, width);
                    if (code == esc) {
                        rk_of[kept] = rk_of[i];
                        ex_of[kept] = ex_of[i];
                        ++kept;
                    }
                }
                w = tier.finish();
                active = kept;
            }
            if (static_cast<uint64_t>(stop - w) != stream_words(active, g.exponent))
                throw std::runtime_error("terminal stream mismatch");
            BitWriter term(w);
            for (uint64_t i = 0; i < active; ++i) term.put(ex_of[i], g.exponent);
            term.finish();
        }
    });
}

// op 2: rows [first, first + nrows), row `first` written at `out`.
template <class T>
void decode(T* out, const Geometry& g, const uint8_t* tables, const uint32_t* offsets, const uint32_t* data,
            uint64_t words, uint64_t first, uint64_t nrows) {
    if (first > g.rows || nrows > g.rows - first || offsets[0] || offsets[g.rows * g.nb] != words)
        throw std::runtime_error("invalid decode range or directory");
    const uint64_t nblocks = nrows * g.nb, base_id = first * g.nb;
    parallel_for(nblocks, 256, [&](uint64_t b, uint64_t e) {
        std::array<uint16_t, kBlock> where;
        for (uint64_t k = b; k < e; ++k) {
            uint64_t id = base_id + k, row = id / g.nb, blk = id % g.nb, n = g.block_len(blk);
            uint64_t pos = offsets[id], end = offsets[id + 1];
            if (end <= pos || end > words) throw std::runtime_error("invalid block bounds");
            T* dst = out + (row - first) * g.cols + blk * kBlock;
            const uint8_t* pal = tables + g.region(row, blk) * g.stride;
            if (stream_words(n, g.mant + 1) > end - pos) throw std::runtime_error("short literal stream");
            BitReader lit(data + pos);
            const uint32_t mmask = (1u << g.mant) - 1;
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t l = lit.get(g.mant + 1);
                dst[i] = static_cast<T>((l & mmask) | ((l >> g.mant) << (g.mant + g.exponent)));
                where[i] = static_cast<uint16_t>(i);
            }
            pos += stream_words(n, g.mant + 1);
            uint64_t active = n;
            for (uint32_t j = 0; j + 1 < g.tiers; ++j) {
                const uint32_t width = g.width[j], esc = (1u << width) - 1;
                const uint64_t len = stream_words(active, width);
                if (len > end - pos) throw std::runtime_error("short exponent stream");
                BitReader tier(data + pos);
                uint64_t kept = 0;
                for (uint64_t i = 0; i < active; ++i) {
                    uint32_t code = tier.get(width);
                    if (code == esc)
                        where[kept++] = where[i];
                    else
                        dst[where[i]] = static_cast<T>(dst[where[i]] | (uint32_t(pal[g.table[j] + code]) << g.mant));
                }
                pos += len;
                active = kept;
            }
            if (stream_words(active, g.exponent) != end - pos) throw std::runtime_error("terminal stream mismatch");
            BitReader term(data + pos);
            for (uint64_t i = 0; i < active; ++i)
                dst[where[i]] = static_cast<T>(dst[where[i]] | (term.get(g.exponent) << g.mant));
        }
    });
}

void fail_into(char* err, uint64_t n, const char* msg) {
    if (err && n) {
        std::strncpy(err, msg, n - 1);
        err[n - 1] = 0;
    }
}

// ---- synthetic data: a counter-based generator ----------------------------

uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Two uniforms in (0, 1] from one 64-bit draw.
void uniforms(uint64_t key, double& u1, double& u2) {
    uint64_t h = mix64(key);
    u1 = (static_cast<double>(h & 0xFFFFFFFFull) + 1.0) * (1.0 / 4294967296.0);
    u2 = (static_cast<double>(h >> 32) + 1.0) * (1.0 / 4294967296.0);
}

uint16_t to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

}  // namespace

extern "C" int dmx_set_host_threads(int n) {
    g_threads.store(n < 0 ? 0 : n);
    return resolve_threads();
}

extern "C" int dmx_radix_native(uint32_t op, void* source_or_output, uint64_t rows, uint64_t cols, uint64_t rg,
                                uint64_t cg, uint32_t mant, uint32_t exponent, const uint32_t* widths,
                                uint32_t count, uint8_t* palettes, uint32_t* offsets, uint32_t* data,
                                uint64_t words, uint64_t first, uint64_t nrows, uint64_t* result, char* error,
                                uint64_t error_size) {
    try {
        const Geometry g(rows, cols, rg, cg, mant, exponent, widths, count);
        const bool wide = exponent == 8;
        switch (op) {
            case 0:
                if (!result) throw std::runtime_error("null result");
                *result = wide ? plan(static_cast<const uint16_t*>(source_or_output), g, palettes, offsets)
                               : plan(static_cast<const uint8_t*>(source_or_output), g, palettes, offsets);
                break;
            case 1:
                if (wide)
                    encode(static_cast<const uint16_t*>(source_or_output), g, palettes, offsets, data, words);
                else
                    encode(static_cast<const uint8_t*>(source_or_output), g, palettes, offsets, data, words);
                break;
            case 2:
                if (wide)
                    decode(static_cast<uint16_t*>(source_or_output), g, palettes, offsets, data, words, first, nrows);
                else
                    decode(static_cast<uint8_t*>(source_or_output), g, palettes, offsets, data, words, first, nrows);
                break;
            case 3:
                rank_tables(g, palettes);
                break;
            default:
                throw std::runtime_error("unknown operation");
        }
        return 0;
    } catch (const std::exception& e) {
        fail_into(error, error_size, e.what());
        return 1;
    }
}

extern "C" int dmx_synth_bf16(uint64_t seed, uint64_t stream, uint64_t count, double scale, uint32_t dist,
                              uint16_t* out, char* err, size_t errn) {
    if (!out && count) {
        fail_into(err, errn, "null output");
        return 1;
    }
    if (dist > 1) {
        fail_into(err, errn, "unknown distribution");
        return 1;
    }
    const uint64_t key = mix64(seed * 0x100000001B3ull ^ mix64(stream + 0x51ED2701ull));
    const double two_pi = 6.283185307179586476925286766559;
    parallel_for(count, 1 << 16, [&](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; ++i) {
            // element pair i / 2 shares one Box-Muller draw
            double u1, u2;
            uniforms(key ^ mix64(i >> 1), u1, u2);
            double rad = std::sqrt(-2.0 * std::log(u1));
            double z = (i & 1) ? rad * std::sin(two_pi * u2) : rad * std::cos(two_pi * u2);
            if (dist == 1) {
                // chi-square with 4 degrees of freedom: -2 ln(u3 u4)
                double u3, u4;
                uniforms(key ^ mix64(i + 0x7F4A7C15F39CC060ull), u3, u4);
                double chi = -2.0 * (std::log(u3) + std::log(u4));
                z = z / std::sqrt(chi / 4.0) / std::sqrt(2.0);
            }
            out[i] = to_bf16(static_cast<float>(z * scale));
        }
    });
    return 0;
}
