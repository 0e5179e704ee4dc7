// Host model of the sip and gulp kernels' reads (test infrastructure).
//
// For each launch configuration it plans the launch with the library's own
// plan_launch (drinkme_amd/csrc/plan.h) and walks every wave of every
// workgroup with the kernels' own cursor functions (wg_place, sip_walk,
// sip_start / sip_next / sip_issue, quad_start / quad_next / quad_issue),
// issuing as many loads past each wave's work as a pipeline may run ahead.
// It checks, for every issue:
//   - the directory index (offsets[blk] and offsets[blk + 1]) lies inside
//     the tensor's R * NB + 1 entries;
//   - an issue on the wave's work is live and names the block the cursor
//     claims: its row partial (slot), its column block among the resident
//     activations, its column phase and whether it closes its unit; an issue
//     past the work (or of a quad row past the tile) reads the workgroup's
//     first block;
// and, per launch, that every block of every row is processed exactly once.
// It also checks the per-lane load offsets against the reach pad.
//
//   walk_model            every configuration; exit status 0 when clean
//   walk_model --plant K  the same with planted mistake K (1..4) in the
//                         walk it models; exit status 0 when the checks
//                         catch it (a negative control)
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "plan.h"

using namespace dmx;

namespace {

int g_plant = 0;
uint64_t g_plans = 0, g_wgs = 0, g_waves = 0, g_blocks = 0, g_issues = 0, g_bad = 0;

void bad(const std::string& what) {
    if (g_bad < 12) fprintf(stderr, "violation: %s\n", what.c_str());
    ++g_bad;
}

// kGulpMatrix / kTwinGulpMatrix: gulp and its twin under the matrix policy
enum Kind { kSip, kGulp, kDecodeSip, kDecodeGulp, kTwinSip, kTwinGulp, kGulpMatrix, kTwinGulpMatrix };
const char* kind_name(Kind k) {
    static const char* n[] = {"sip",      "gulp",      "decode-sip",  "decode-gulp",
                              "twin-sip", "twin-gulp", "gulp-matrix", "twin-gulp-matrix"};
    return n[k];
}

struct Case {
    Kind kind;
    std::vector<uint32_t> rows;
    uint32_t cols, m, cus;
};

std::string describe(const Case& c) {
    std::string s = std::string(kind_name(c.kind)) + " rows";
    for (uint32_t r : c.rows) s += " " + std::to_string(r);
    return s + " cols " + std::to_string(c.cols) + " m " + std::to_string(c.m) + " cus " + std::to_string(c.cus);
}

// The launch parameters each kernel's host code passes to plan_launch.
struct Launch {
    uint32_t per_cu;
    bool quad, allow_two, gulp;
    double unit_cost;
    size_t fixed;
};

Launch launch_of(Kind k, uint32_t M) {
    Launch l{};
    const bool matrix = k == kGulpMatrix || k == kTwinGulpMatrix;
    l.gulp = k == kGulp || k == kDecodeGulp || k == kTwinGulp || matrix;
    const bool dec = k == kDecodeSip || k == kDecodeGulp;
    l.per_cu = dec ? kDecodePerCu : l.gulp ? gulp_per_cu((int)M, matrix) : kSipPerCu;
    l.quad = dec ? false : l.gulp ? gulp_quad((int)M, matrix) : sip_quad((int)M);
    l.allow_two = !l.gulp;
    l.unit_cost = unit_end_cost(l.gulp, (int)M, dec, matrix);
    l.fixed = l.gulp ? kGulpStaticLds : kSipStaticLds;
    return l;
}

// One launch: plan, walk, check. Returns false when no plan fits (the host
// then runs the generic kernel, which has no cursor).
template <bool TWO>
void walk_launch(const Case& cs, const SipShape& sh, const uint32_t (&row0)[kGroupMax + 1], uint32_t grid) {
    const uint32_t W = sh.waves;
    std::vector<uint8_t> seen((size_t)sh.rows * sh.nb, 0);
    const std::string tag = describe(cs);
    for (uint32_t wg = 0; wg < grid; ++wg) {
        ++g_wgs;
        const WgPlace wp = wg_place<TWO>(sh, row0, wg);
        if (wp.nrows == 0 || wp.r0 + wp.nrows > sh.rows) {
            bad(tag + ": workgroup " + std::to_string(wg) + " outside the rows");
            continue;
        }
        if (!TWO && wp.split != wp.nrows) bad(tag + ": a tile spans two tensors without TWO");
        const uint32_t urows = unit_rows(sh, wp.nrows);
        const uint32_t units = urows * sh.segs;
        const SipWalk wk = sh.quad ? sip_walk<true>(sh, wp.nrows) : sip_walk<false>(sh, wp.nrows);
        for (uint32_t wv = 0; wv < W; ++wv) {
            ++g_waves;
            const uint32_t my_units = wv < units ? (units - wv + W - 1) / W : 0;
            const uint32_t items = my_units * sh.seg_blocks * (sh.quad ? 4 : 1);
            SipCursor c{};
            QuadCursor q{};
            if (sh.quad)
                quad_start(sh, q, wv, wk);
            else
                sip_start<TWO>(sh, c, wv, wk, wp.sp);
            for (uint32_t k = 0; k < items + 8; ++k) {
                ++g_issues;
                Issue is;
                uint32_t slot = 0, cb = 0, ph = 0, trow = 0;
                bool last = false, quad_live_row = true;
                if (sh.quad) {
                    is = quad_issue<TWO>(sh, q, wp.sp, wp.nrows);
                    trow = 4 * q.q + q.sub;
                    quad_live_row = trow < wp.nrows;
                    cb = q.sp * sh.seg_blocks + q.c;
                    ph = q.p;
                    slot = trow * sh.segs + q.p * sh.psegs + q.sp;
                    last = q.c + 1 == sh.seg_blocks;
                } else {
                    is = sip_issue<TWO>(sh, c, wp.sp);
                    cb = c.cb;
                    ph = c.p;
                    slot = c.slot;
                    last = c.j + 1 == sh.seg_blocks;
                }
                // planted mistakes (negative controls of this model)
                if (g_plant == 1 && k == items && items) is.blk = is.live ? is.blk : is.blk + sh.nb * 64;  // past work reads beyond
                if (g_plant == 3 && wg == grid / 2 && wv == 0 && k == 0 && items) slot += 1;           // wrong partial
                const uint32_t tt = is.t ? wp.ib : wp.ia;
                const uint32_t tblocks = cs.rows[tt] * sh.nb;
                if (is.blk >= tblocks)
                    bad(tag + ": directory index " + std::to_string(is.blk) + " past " + std::to_string(tblocks) +
                        " blocks (wg " + std::to_string(wg) + " wave " + std::to_string(wv) + ")");
                const uint32_t grow = row0[tt] + is.blk / sh.nb, cbg = is.blk % sh.nb;
                const uint32_t r = grow - wp.r0;  // the block's place in the tile, from its directory index
                if (k < items && quad_live_row && !is.live) {
                    bad(tag + ": an issue on the wave's work is not live");
                } else if (k < items && quad_live_row && (grow < wp.r0 || r >= wp.nrows)) {
                    bad(tag + ": a block of another tile");
                } else if (k < items && quad_live_row) {
                    if (sh.quad && r != trow) bad(tag + ": quad row mismatch");
                    const uint32_t K = sh.phase_blocks, L = sh.seg_blocks;
                    if (slot != r * sh.segs + cbg / L) bad(tag + ": wrong row partial");
                    if (cb != cbg % K || ph != cbg / K) bad(tag + ": wrong column block or phase");
                    if (last != (cbg % L == L - 1)) bad(tag + ": wrong unit end");
                    // the gulp kernel's rare paths rebuild the block from the
                    // unit and column
                    if (!TWO && !sh.quad && row_block(sh, c, wp.sp) != is.blk) bad(tag + ": row_block != c.blk");
                    const size_t idx = (size_t)grow * sh.nb + cbg;
                    if (g_plant != 4 || idx != 0) ++seen[idx];
                    ++g_blocks;
                } else {
                    if (is.live || is.blk != wp.sp.a_first || is.t != 0)
                        bad(tag + ": an issue past the work does not read the workgroup's first block");
                }
                if (sh.quad) {
                    quad_next(sh, q, wk);
                } else {
                    sip_next<TWO>(sh, c, wk, wp.sp);
                    if (g_plant == 2 && k == 0 && wg == 0 && wv == 0) c.blk += 1;  // a skipped block
                }
            }
        }
    }
    for (size_t i = 0; i < seen.size(); ++i)
        if (seen[i] != 1) {
            bad(tag + ": block " + std::to_string(i) + " processed " + std::to_string(seen[i]) + " times");
            break;
        }
}

void run(const Case& cs) {
    const uint32_t n = (uint32_t)cs.rows.size();
    const uint32_t mi = cs.m == 1 ? 0 : cs.m == 2 ? 1 : cs.m <= 4 ? 2 : 3;
    const uint32_t M = 1u << mi;
    const Launch l = launch_of(cs.kind, M);
    SipShape sh{};
    uint32_t row0[kGroupMax + 1];
    uint64_t total = 0;
    uint32_t min_rows = cs.rows[0];
    for (uint32_t i = 0; i < (uint32_t)kGroupMax; ++i) {
        row0[i] = (uint32_t)total;
        if (i < n) {
            total += cs.rows[i];
            min_rows = std::min(min_rows, cs.rows[i]);
        }
    }
    row0[kGroupMax] = (uint32_t)total;
    for (uint32_t i = n; i <= (uint32_t)kGroupMax; ++i) row0[i] = (uint32_t)total;
    sh.rows = (uint32_t)total;
    sh.cols = cs.cols;
    sh.nb = cs.cols / 1024;
    sh.n = n;
    sh.m = cs.m;
    uint32_t grid = 0;
    size_t lds = 0;
    bool two = false;
    // (the gulp GEMV plans through plan_gulp, as its launcher does)
    if (cs.kind == kGulp || cs.kind == kGulpMatrix
            ? !plan_gulp(sh, row0, n, min_rows, M, cs.cus, grid, lds, two, cs.kind == kGulpMatrix)
                         : !plan_launch(sh, row0, n, min_rows, M, kPlanWaves, l.per_cu, l.quad, l.unit_cost, l.fixed,
                                        l.allow_two, cs.cus, grid, lds, two))
        return;  // the generic kernel runs
    const bool dec = cs.kind == kDecodeSip || cs.kind == kDecodeGulp;
    if (dec && sh.phases > 1) return;  // the decode runs unphased, else generic
    ++g_plans;
    const std::string tag = describe(cs);
    if ((lds + l.fixed) > kLdsBytes) bad(tag + ": LDS past the CU's");
    if (sh.segs * sh.seg_blocks != sh.nb || sh.phases * sh.phase_blocks != sh.nb) bad(tag + ": segments do not tile the row");
    if (sh.quad && sh.rows_per_wg % 4) bad(tag + ": a quad tile of " + std::to_string(sh.rows_per_wg) + " rows");
    if ((cs.kind == kTwinSip || cs.kind == kTwinGulp || cs.kind == kTwinGulpMatrix) &&
        (uint64_t)sh.rows_per_wg * cs.cols * 2 >= (1ull << 31))
        return;  // the host refuses the fast twin
    if (two)
        walk_launch<true>(cs, sh, row0, grid);
    else
        walk_launch<false>(cs, sh, row0, grid);
}

// The per-lane loads against the reach pad (block_word_bounds(1024)[1]):
// sip 608 words, gulp 768.
void check_reach() {
    uint32_t sip_end = 0, gulp_end = 0;
    for (uint32_t lane = 0; lane < 64; ++lane) {
        const SipLanes s = sip_lanes(lane);
        sip_end = std::max({sip_end, s.lit + kSipLitBytes, s.t0 + kSipT0Bytes, s.term + kSipTermBytes});
        const GulpLanes g = gulp_lanes(lane);
        // literal plane, tier-0 word, tail word (tier 1, tier 2, terminal)
        gulp_end = std::max({gulp_end, g.lit + 16, 4 * 256 + g.w + 4, 4 * kGulpFixed + g.w + 4});
    }
    if (sip_end > 4 * 608 || gulp_end > 4 * 768) bad("a lane's load reaches past the pad");
    printf("reach: sip loads end %u words past a block's start (pad 608), gulp %u (pad 768)\n", sip_end / 4,
           gulp_end / 4);
}

uint64_t g_rng = 0x9E3779B97F4A7C15ull;
uint32_t rnd(uint32_t n) {
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (uint32_t)(g_rng % n);
}

}  // namespace

// gulp's tier-1 table (625 entries in LDS, no bounds check on its reads):
// every (m0, codes) the kernel can look up, codes < 4^popcount(m0), lies
// in the table, each entry is one pair's, and the table build's inverse
// maps each entry back to its pair.
void check_gulp_t1() {
    std::vector<int> hit(kGulpT1Entries, 0);
    for (uint32_t m0 = 0; m0 < 16; ++m0)
        for (uint32_t c = 0; c < (1u << (2 * __builtin_popcount(m0))); ++c) {
            const uint32_t i = gulp_t1_base(m0) + c;
            if (i >= kGulpT1Entries) {
                bad("gulp tier-1 index " + std::to_string(i) + " past the table");
                continue;
            }
            ++hit[i];
            uint32_t m, k;
            gulp_t1_entry(i, m, k);
            if (m != m0 || k != c) bad("gulp tier-1 entry " + std::to_string(i) + " maps back wrong");
        }
    for (uint32_t i = 0; i < kGulpT1Entries; ++i)
        if (hit[i] != 1) bad("gulp tier-1 entry " + std::to_string(i) + " held by " + std::to_string(hit[i]));
}

// gulp's tables as the kernel looks them up, against a direct decode of
// the codes: for seeded palettes, every tier-0 pattern and every tier-1 code
// pattern of its escapes, the codes placed at an even offset of a random
// window. The exponent fields of tier 0 | tier 1 must be the palette entries
// at the positions that do not escape twice, zero at those that do; m1 and
// its count must name those; the tier-1 bit count must be 2 popcount(m0).
// (Planted mistake 5: the runs' byte offsets at 16 bytes an entry.)
void check_gulp_tables() {
    uint64_t rng = 0x243F6A8885A308D3ull;
    auto next = [&]() {
        rng = rng * 6364136223846793005ull + 1442695040888963407ull;
        return (uint32_t)(rng >> 32);
    };
    for (int pal = 0; pal < 64; ++pal) {
        const uint32_t p0 = next() & 0x00FFFFFFu, p1 = next() & 0x00FFFFFFu;  // byte 3: the escape's zero
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t f[4];
            gulp_t0_entry(p0, i, f);
            if (g_plant == 5) f[3] *= 2;
            uint32_t m0 = 0;
            for (uint32_t k = 0; k < 4; ++k) m0 |= (uint32_t)(((i >> (2 * k)) & 3u) == 3u) << k;
            const uint32_t n1 = (uint32_t)__builtin_popcount(m0);
            if (f[2] != 2 * n1) bad("gulp tier-0 entry " + std::to_string(i) + ": tier-1 bit count");
            for (uint32_t codes = 0; codes < (1u << (2 * n1)); ++codes) {
                const uint32_t off = 2 * (next() % (17 - n1));  // the group's bits end by bit 32
                uint32_t w1 = next();
                if (n1) w1 = (w1 & ~(((1u << (2 * n1)) - 1u) << off)) | (codes << off);
                const uint32_t byte = gulp_t1_byte(w1, off, f[2], f[3]);
                if (byte % 8 || byte / 8 >= kGulpT1Entries) {
                    bad("gulp tier-1 lookup " + std::to_string(byte) + " outside the table");
                    continue;
                }
                uint32_t v[2];
                gulp_t1_value(p1, byte / 8, v);
                uint32_t want[2] = {0, 0}, m1 = 0, r = 0;
                for (uint32_t k = 0; k < 4; ++k) {
                    const uint32_t c0 = (i >> (2 * k)) & 3u;
                    uint32_t e = (p0 >> (8 * c0)) & 0xFFu;
                    if (c0 == 3u) {
                        const uint32_t c1 = (codes >> (2 * r++)) & 3u;
                        e = c1 == 3u ? 0u : (p1 >> (8 * c1)) & 0xFFu;
                        m1 |= (uint32_t)(c1 == 3u) << k;
                    }
                    want[k / 2] |= e << (k % 2 ? 23 : 7);
                }
                const uint32_t ex = 0x7F807F80u;
                if (((f[0] | v[0]) & ex) != want[0] || ((f[1] | v[1]) & ex) != want[1] ||
                    ((v[0] >> 3) & 15u) != m1 || ((v[0] >> 15) & 7u) != (uint32_t)__builtin_popcount(m1)) {
                    bad("gulp tables: tier-0 pattern " + std::to_string(i) + ", tier-1 codes " +
                        std::to_string(codes) + " decode wrong");
                    return;
                }
            }
        }
    }
}

int main(int argc, char** argv) {
    if (argc == 3 && !strcmp(argv[1], "--plant")) g_plant = atoi(argv[2]);
    check_reach();
    check_gulp_t1();
    check_gulp_tables();
    // the configurations' launches: Qwen3-8B (q/k/v, o, gate/up, down,
    // lm_head) and the 32B class, grouped as the benchmark groups them
    const std::vector<std::pair<std::vector<uint32_t>, uint32_t>> shapes = {
        {{4096}, 4096},         {{4096, 1024, 1024}, 4096}, {{12288, 12288}, 4096}, {{4096}, 12288},
        {{151936}, 4096},       {{8192, 1024, 1024}, 5120}, {{5120}, 8192},          {{25600, 25600}, 5120},
        {{5120}, 25600},        {{1024}, 4096},             {{1}, 1024},             {{3, 5, 7, 9}, 2048},
        {{1000, 24, 3000}, 3072}};
    const Kind kinds[] = {kSip, kGulp, kDecodeSip, kDecodeGulp, kTwinSip, kTwinGulp, kGulpMatrix, kTwinGulpMatrix};
    for (const auto& s : shapes)
        for (Kind k : kinds)
            for (uint32_t m : {1u, 2u, 3u, 4u, 5u, 8u})
                for (uint32_t cus : {256u, 80u, 7u}) {
                    if ((k == kDecodeSip || k == kDecodeGulp || k == kTwinSip || k == kTwinGulp ||
                         k == kTwinGulpMatrix) &&
                        (s.first.size() > 1 || ((k == kDecodeSip || k == kDecodeGulp) && m > 1)))
                        continue;
                    run(Case{k, s.first, s.second, m, cus});
                }
    // seeded random groups
    for (int i = 0; i < 600; ++i) {
        Case c;
        const Kind k = i % 3 == 2 ? kGulpMatrix : kinds[rnd(2)];
        c.kind = k;
        const uint32_t n = 1 + rnd(4);
        for (uint32_t j = 0; j < n; ++j) c.rows.push_back(rnd(4) == 0 ? 1 + rnd(40) : 1 + rnd(20000));
        c.cols = 1024 * (1 + rnd(25));
        c.m = 1 + rnd(8);
        static const uint32_t cus[] = {256, 80, 7, 1};
        c.cus = cus[rnd(4)];
        run(c);
    }
    printf("walk model: %llu plans, %llu workgroups, %llu waves, %llu issues, %llu blocks processed; %llu violations\n",
           (unsigned long long)g_plans, (unsigned long long)g_wgs, (unsigned long long)g_waves,
           (unsigned long long)g_issues, (unsigned long long)g_blocks, (unsigned long long)g_bad);
    if (g_plant) {
        printf("planted mistake %d: %s\n", g_plant, g_bad ? "caught" : "NOT caught");
        return g_bad ? 0 : 1;
    }
    return g_bad ? 1 : 0;
}
