// The launch plan and the unit walk of the sip and gulp GEMV kernels
// (kernels.hip), in one header that the kernels and a host model of their
// reads both compile: the model (tests/walk_model.cpp) runs these same
// functions over every workgroup and wave of a plan and checks that every
// directory and schedule index a launch reads lies inside its arrays and
// that every block of every row is processed exactly once, into the right
// partial sum.
//
// Work split. A launch covers the rows of a group of tensors (one row space,
// tensor i from row0[i]); workgroup g owns rows [g T, g T + T). Each row is
// cut into S = P * psegs segments of L = NB / S column blocks, P being the
// column phases (the activation slices resident in LDS in turn). The units
// of a workgroup are dealt to its W waves round-robin, phase-major:
//   row mode   unit (p, r, sp) = row r's blocks of segment p psegs + sp;
//   quad mode  unit (p, q, sp) = the same segment of rows 4q .. 4q + 3,
//              column by column, the four rows' blocks in turn (the matrix
//              core verify rows contract four output rows at once; a row
//              past the tile's end reads a valid block whose sums are
//              never stored).
// A wave walks its units with additions only (dp, dr, ds: a step of W
// units), and a cursor past its last unit (p >= P) reads the workgroup's
// first block, so a load pipeline may run ahead of the work.
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __HIPCC__
#define DMX_HD __host__ __device__ __forceinline__
#define DMX_UNROLL _Pragma("unroll")
#else
#define DMX_HD inline
#define DMX_UNROLL
#endif

#include <algorithm>
#include <cmath>
#include <numeric>

namespace dmx {

constexpr int kGroupMax = 4;          // tensors per grouped launch
constexpr uint32_t kPlanWaves = 12;   // waves per workgroup of the sip and gulp kernels
constexpr uint32_t kGulpWaves3 = 8;   // gulp's waves per workgroup at three workgroups per CU
static_assert(kGulpWaves3 * 64 >= 256 && kPlanWaves * 64 >= 256, "the gulp tables take one entry a thread");
constexpr uint32_t kSipFixed = 256 + 96;   // sip: literal plane + tier-0 words of a 1024-weight block
constexpr uint32_t kGulpFixed = 256 + 64;  // gulp: literal plane + tier-0 words
constexpr uint32_t kTableBytes = 4096 * 8;  // one sip exponent table (a second one for a tile spanning two tensors)
constexpr size_t kLdsBytes = 160 * 1024;    // LDS of one CU

// Resident workgroups per CU that the plans aim for. sip: one. Its loads
// fill the CU's memory path with 12 waves; a second workgroup starts
// behind the first (its activation loads queue behind the first's payload
// misses) and only adds dispatch and setup: one per CU measured 2% faster
// on the Qwen3-8B step and 12% on 4096 x 4096 GEMVs. gulp: two, as its
// decode is bound by instruction latency and needs the waves. The decode
// mode (2 KB stored per block): two, measured 3-11% faster than one.
constexpr uint32_t kSipPerCu = 1, kGulpPerCu = 2, kDecodePerCu = 2;

// Static LDS of the sip and gulp kernels (their tables), for the plans: sip
// its 4096-entry exponent table, its selector tables and its progress
// counter (4 bytes, 16 with alignment); gulp its tier-0 and tier-1 tables,
// selectors, the tier-2 palette and each wave's exponent byte exchange.
constexpr uint32_t kSelBytes = (16 + 13 * 16) * 8;
constexpr uint32_t kGulpT0Bytes = 256 * 16;
// gulp's tier-1 table: for each tier-0 escape mask m0 of a group of four
// weights, a run of 4^popcount(m0) entries (its tier-1 code patterns), the
// runs in order of m0: 625 entries of 8 bytes. m0's run starts after those
// of the masks below it; the ones that first differ from m0 at its set bit
// k are 2^k masks with 4^popcount(m0 above k) 5^k patterns in all.
DMX_HD constexpr uint32_t gulp_t1_base(uint32_t m0) {
    uint32_t b = 0, p5 = 1;
    for (uint32_t k = 0; k < 5; ++k, p5 *= 5)
        if ((m0 >> k) & 1u) b += p5 << (2 * __builtin_popcount(m0 >> (k + 1)));
    return b;
}
constexpr uint32_t kGulpT1Entries = 625;
static_assert(gulp_t1_base(16) == kGulpT1Entries, "the runs of the gulp tier-1 table");
// the inverse: entry i < 625 of the table is m0's entry `codes` (a running
// sum over the runs, at most 16 steps)
DMX_HD void gulp_t1_entry(uint32_t i, uint32_t& m0, uint32_t& codes) {
    uint32_t base = 0, run = 1;
    m0 = 0;
    while (i >= base + run) {
        base += run;
        run = 1u << (2 * __builtin_popcount(++m0));
    }
    codes = i - base;
}

// The gulp tables' entries, built by the kernels in LDS from the palette's
// tier-0 word p0 and tier-1 word p1 (bytes 0..2 the entries, byte 3 the
// zero that an escape code reads).
// Tier-0 entry i, four 2-bit codes c_k = (i >> 2k) & 3: E(c0) << 7 |
// E(c1) << 23, E(c2) << 7 | E(c3) << 23 (the bf16 pairs' exponent fields),
// 2 popcount(m0) and 8 t1_base(m0), m0 the positions whose code is 3.
DMX_HD void gulp_t0_entry(uint32_t p0, uint32_t i, uint32_t (&f)[4]) {
    uint32_t e[4], m = 0;
    for (uint32_t k = 0; k < 4; ++k) {
        const uint32_t c = (i >> (2 * k)) & 3u;
        e[k] = (p0 >> (8 * c)) & 0xFFu;
        m |= (uint32_t)(c == 3u) << k;
    }
    f[0] = (e[0] << 7) | (e[1] << 23);
    f[1] = (e[2] << 7) | (e[3] << 23);
    f[2] = 2u * (uint32_t)__builtin_popcount(m);
    f[3] = 8u * gulp_t1_base(m);
}
// Tier-1 entry i (m0's entry `codes`): its popcount(m0) codes, 2 bits each
// in order, at the positions of m0, as the same exponent pairs, with m1 (the
// positions whose tier-1 code is 3) << 3 | popcount(m1) << 15 in the first.
DMX_HD void gulp_t1_value(uint32_t p1, uint32_t i, uint32_t (&v)[2]) {
    uint32_t m0, codes;
    gulp_t1_entry(i, m0, codes);
    uint32_t e[4], m1 = 0, r = 0;
    for (uint32_t k = 0; k < 4; ++k) {
        e[k] = 0;
        if ((m0 >> k) & 1u) {
            const uint32_t c = (codes >> (2 * r++)) & 3u;
            e[k] = (p1 >> (8 * c)) & 0xFFu;
            m1 |= (uint32_t)(c == 3u) << k;
        }
    }
    v[0] = (e[0] << 7) | (e[1] << 23) | (m1 << 3) | ((uint32_t)__builtin_popcount(m1) << 15);
    v[1] = (e[2] << 7) | (e[3] << 23);
}
// A group's tier-1 entry, as a byte offset in the table: its f2 = 2
// popcount(m0) code bits from bit `off` of the lane's tier-1 window w1 (a
// v_bfe: width 0 reads 0), in the run at byte f3 (f2, f3: its tier-0 entry's)
DMX_HD uint32_t gulp_t1_byte(uint32_t w1, uint32_t off, uint32_t f2, uint32_t f3) {
#ifdef __HIP_DEVICE_COMPILE__
    return (__builtin_amdgcn_ubfe(w1, off, f2) << 3) + f3;
#else
    return ((f2 ? (w1 >> off) & (0xFFFFFFFFu >> (32 - f2)) : 0u) << 3) + f3;
#endif
}
constexpr uint32_t kGulpX2Words = 40;  // per wave: 128 exponent bytes + a window's overhang
constexpr size_t kSipStaticLds = kTableBytes + kSelBytes + 16;
constexpr size_t kGulpStaticLds = kGulpT0Bytes + ((kGulpT1Entries * 8 + 15) & ~15u) + 13 * 16 * 8 + 16 + kPlanWaves * kGulpX2Words * 4;

// Verify rows in quad units: four output rows contracted at once on the
// matrix cores, sip at M = 4 and 8, gulp at M = 8. The quad path holds four
// decoded blocks in registers, so a gulp launch of it runs one workgroup
// per CU; gulp's decode is bound by latency and wants the waves of two, so
// at M = 4 it keeps v_dot2 (the quad path measured 4-13% slower there on
// Qwen3-8B and 32B-class layers, and 4-8% faster at M = 8).
// The matrix policy (DMX_POLICY_MATRIX) also puts gulp's 4-row verify in
// quad units, so that path can be chosen and measured.
DMX_HD constexpr bool sip_quad(int M) { return M >= 4; }
DMX_HD constexpr bool gulp_quad(int M, bool matrix = false) { return M >= 8 || (matrix && M == 4); }
DMX_HD constexpr uint32_t gulp_per_cu(int M, bool matrix = false) { return gulp_quad(M, matrix) ? 1u : kGulpPerCu; }

struct SipShape {
    uint32_t rows, cols, nb;  // rows of the whole group
    uint32_t n;               // tensors in the group
    uint32_t rows_per_wg;     // T
    uint32_t segs;            // S (segments per row) = phases * psegs
    uint32_t seg_blocks;      // L = NB / S
    uint32_t phases;          // P: column phases (1 = every activation column resident in LDS)
    uint32_t phase_blocks;    // K = NB / P column blocks of activations in LDS at a time
    uint32_t xrow;            // LDS stride of the activation rows, in bf16: K * 1024 plus a bank-spreading pad
    uint32_t waves;           // W: waves per workgroup
    uint32_t psegs;           // segments per phase
    uint32_t quad;            // 1: quad-mode units (four rows at once)
    uint32_t dp, dr, ds;      // a wave's step of W units in a full tile: phases, rows (quads), segments
    uint32_t tbl2_lds;        // dynamic-LDS byte offset of the second table; 0 = no workgroup spans two tensors
    uint32_t young_from;      // first workgroup dispatched as a CU's second (~0u: one per CU)
    uint32_t m;               // activation rows (<= the kernel's M; rows past m are padding)
    int bias_dtype, out_dtype;
};

// Unit rows of a tile of nrows rows: rows, or quads of four.
DMX_HD uint32_t unit_rows(const SipShape& sh, uint32_t nrows) { return sh.quad ? (nrows + 3) / 4 : nrows; }

// A wave's place in its work (row mode): block j of the unit, the block's
// index in its tensor's directory, its column block among the resident
// activation columns, and which of the workgroup's tensors it belongs to.
struct SipCursor {
    uint32_t j, blk, cb, t;
    uint32_t p, r, sp;  // the unit: column phase, row of the workgroup, segment within the phase
    uint32_t slot;      // the unit's row partial: row * S + segment
};

// Quad mode: the unit (p, q, sp), the block's column c in the segment and
// row sub in the quad, and wb0, the workgroup block index of (row 4q,
// column 0 of the segment).
struct QuadCursor {
    uint32_t p, q, sp;
    uint32_t c, sub;
    uint32_t wb0;
};

// The workgroup's blocks in row-major order: [0, split_blocks) are its
// first tensor's, from that tensor's block a_first; the rest its second
// tensor's, from block 0.
struct SipSpan {
    uint32_t a_first, split_blocks;
};

// A wave's step of W units over a tile of nrows unit rows.
struct SipWalk {
    uint32_t nrows, dp, dr, ds;
};

// Where workgroup wg sits in the group: its first row r0 and row count,
// the tensor ia holding r0 and the next one ib, their first rows, and the
// tile's split into ia's rows [0, split) and ib's [split, nrows).
struct WgPlace {
    uint32_t r0, nrows, ia, ib, row_a, row_b, split, lrow_a;
    SipSpan sp;
};

template <bool TWO>
DMX_HD WgPlace wg_place(const SipShape& sh, const uint32_t (&row0)[kGroupMax + 1], uint32_t wg) {
    WgPlace w;
    w.r0 = wg * sh.rows_per_wg;
    w.nrows = sh.rows - w.r0 < sh.rows_per_wg ? sh.rows - w.r0 : sh.rows_per_wg;
    uint32_t ia = 0;
    DMX_UNROLL
    for (int i = 1; i < kGroupMax; ++i) ia += (uint32_t)i < sh.n && row0[i] <= w.r0;
    w.ia = ia;
    w.ib = ia + 1 < sh.n - 1 ? ia + 1 : sh.n - 1;
    uint32_t row_a = row0[0], row_b = row0[1];
    DMX_UNROLL
    for (int k = 1; k < kGroupMax; ++k) {
        row_a = ia == (uint32_t)k ? row0[k] : row_a;
        row_b = ia == (uint32_t)k ? row0[k + 1] : row_b;
    }
    w.row_a = row_a;
    w.row_b = row_b;
    const uint32_t end = w.r0 + w.nrows;
    w.split = TWO ? (row_b < end ? row_b : end) - w.r0 : w.nrows;
    w.lrow_a = w.r0 - row_a;
    w.sp.a_first = w.lrow_a * sh.nb;
    w.sp.split_blocks = w.split * sh.nb;
    return w;
}

template <bool QUAD>
DMX_HD SipWalk sip_walk(const SipShape& sh, uint32_t nrows) {
    SipWalk w;
    w.nrows = QUAD ? (nrows + 3) / 4 : nrows;
    if (nrows == sh.rows_per_wg) {  // every tile but perhaps the last: the host's step
        w.dp = sh.dp;
        w.dr = sh.dr;
        w.ds = sh.ds;
    } else {
        const uint32_t pu = w.nrows * sh.psegs, rem = sh.waves % pu;
        w.dp = sh.waves / pu;
        w.dr = rem / sh.psegs;
        w.ds = rem - w.dr * sh.psegs;
    }
    return w;
}

// Advances a unit (p, r, sp) by the walk's step of W units.
DMX_HD void unit_step(const SipShape& sh, const SipWalk& w, uint32_t& p, uint32_t& r, uint32_t& sp) {
    p += w.dp;
    r += w.dr;
    sp += w.ds;
    if (sp >= sh.psegs) {
        sp -= sh.psegs;
        ++r;
    }
    if (r >= w.nrows) {
        r -= w.nrows;
        ++p;
    }
}

// Unit u (< W: a wave's first unit), counted up from unit 0.
DMX_HD void unit_at(const SipShape& sh, const SipWalk& w, uint32_t u, uint32_t& p, uint32_t& r, uint32_t& sp) {
    p = r = sp = 0;
    for (uint32_t i = 0; i < u; ++i) {
        if (++sp == sh.psegs) {
            sp = 0;
            if (++r == w.nrows) {
                r = 0;
                ++p;
            }
        }
    }
}

// ---- row mode

// Sets the block fields of the cursor's unit.
template <bool TWO>
DMX_HD void sip_unit(const SipShape& sh, SipCursor& c, const SipSpan& sp) {
    c.j = 0;
    const uint32_t seg = c.p * sh.psegs + c.sp;
    c.slot = c.r * sh.segs + seg;
    const uint32_t wb = c.r * sh.nb + seg * sh.seg_blocks;
    c.cb = c.sp * sh.seg_blocks;
    c.t = TWO && wb >= sp.split_blocks;
    c.blk = c.t ? wb - sp.split_blocks : sp.a_first + wb;
}

template <bool TWO>
DMX_HD void sip_start(const SipShape& sh, SipCursor& c, uint32_t u, const SipWalk& w, const SipSpan& sp) {
    unit_at(sh, w, u, c.p, c.r, c.sp);
    sip_unit<TWO>(sh, c, sp);
}

template <bool TWO>
DMX_HD void sip_next(const SipShape& sh, SipCursor& c, const SipWalk& w, const SipSpan& sp) {
    if (++c.j == sh.seg_blocks) {
        unit_step(sh, w, c.p, c.r, c.sp);
        sip_unit<TWO>(sh, c, sp);
    } else {
        ++c.blk;
        ++c.cb;
    }
}

// A one-tensor row-mode cursor's block rebuilt from its unit and column
// (c.blk while the cursor is on the wave's work), for code that keeps those
// live but not c.blk.
DMX_HD uint32_t row_block(const SipShape& sh, const SipCursor& c, const SipSpan& sp) {
    return sp.a_first + c.r * sh.nb + c.p * sh.psegs * sh.seg_blocks + c.cb;
}

// The block a row-mode issue reads: the cursor's while it is on the wave's
// work, else the workgroup's first block (of its first tensor).
struct Issue {
    uint32_t blk, t;
    bool live;
};

template <bool TWO>
DMX_HD Issue sip_issue(const SipShape& sh, const SipCursor& c, const SipSpan& sp) {
    Issue is;
    is.live = c.p < sh.phases;
    is.t = TWO && is.live ? c.t : 0u;
    is.blk = is.live ? c.blk : sp.a_first;
    return is;
}

// ---- quad mode

DMX_HD void quad_unit(const SipShape& sh, QuadCursor& c) {
    c.c = c.sub = 0;
    c.wb0 = 4 * c.q * sh.nb + (c.p * sh.psegs + c.sp) * sh.seg_blocks;
}

DMX_HD void quad_start(const SipShape& sh, QuadCursor& c, uint32_t u, const SipWalk& w) {
    unit_at(sh, w, u, c.p, c.q, c.sp);
    quad_unit(sh, c);
}

DMX_HD void quad_next(const SipShape& sh, QuadCursor& c, const SipWalk& w) {
    if (++c.sub == 4) {
        c.sub = 0;
        if (++c.c == sh.seg_blocks) {
            unit_step(sh, w, c.p, c.q, c.sp);
            quad_unit(sh, c);
        }
    }
}

// The block a quad-mode issue reads: row 4q + sub of the tile at the
// cursor's column, else (past the wave's work, or a row past the tile's
// end) the workgroup's first block.
template <bool TWO>
DMX_HD Issue quad_issue(const SipShape& sh, const QuadCursor& c, const SipSpan& sp, uint32_t nrows) {
    Issue is;
    is.live = c.p < sh.phases && 4 * c.q + c.sub < nrows;
    const uint32_t wb = c.wb0 + c.sub * sh.nb + c.c;
    const bool tb = TWO && wb >= sp.split_blocks;
    is.t = is.live && tb ? 1u : 0u;
    is.blk = !is.live ? sp.a_first : tb ? wb - sp.split_blocks : sp.a_first + wb;
    return is;
}

// ---- the per-lane loads of a block

// sip: byte offsets from the block's first word of lane l's three loads:
// its 16 literal bytes (weights 16l .. 16l + 15), the two tier-0 words
// holding its sixteen 3-bit codes (48 bits at bit 48l) and word l of the
// terminal; the raw twin's 32 bytes of the lane's bf16 weights.
struct SipLanes {
    uint32_t lit, t0, term;
    uint32_t raw;
};

DMX_HD SipLanes sip_lanes(uint32_t lane) {
    SipLanes ln;
    ln.lit = 16 * lane;
    ln.t0 = 4 * 256 + 4 * ((3 * lane) >> 1);
    ln.term = 4 * (kSipFixed + lane);
    ln.raw = 32 * lane;
    return ln;
}
constexpr uint32_t kSipLitBytes = 16, kSipT0Bytes = 8, kSipTermBytes = 4;

// gulp: 16 literal bytes (lit); tier-0 word l and tail word l (w, plus
// the constant starts 256 and 320 words; the tail holds tier 1, tier 2 and
// the terminal back to back). t2: the byte address, among the tail's lanes,
// of lane l's tier-2 word l / 4 (from the tier-2 start w1).
struct GulpLanes {
    uint32_t lit, w, t2;
};

DMX_HD GulpLanes gulp_lanes(uint32_t lane) {
    GulpLanes ln;
    ln.lit = 16 * lane;
    ln.w = 4 * lane;
    ln.t2 = 4 * (lane >> 2);
    return ln;
}

// ---- the plan (host)

// What the planner charges a unit's end, per activation row, in blocks: a
// quarter for sip, for the quad units and for the decode (which stores its
// blocks and sums nothing); a whole block for gulp's v_dot2 path, whose
// blocks are bound by instruction issue and whose unit end (the wave's
// sum, its LDS write and the cursor's step) is some 60 instructions: with
// it the Qwen3-8B q/k/v and o run whole rows as units (the Qwen3-8B gulp
// layer 1.1-1.4% faster at M = 1 and 1.0-2.1% at M = 4, the 32B-class
// layer 0.5-1.9% at M = 1, over two A/B runs); charging the quad units so
// made M = 8 9% slower.
DMX_HD constexpr double unit_end_cost(bool gulp, int M, bool decode, bool matrix = false) {
    return gulp && !decode && !gulp_quad(M, matrix) ? 1.0 : 0.25;
}

// The work plan of a sip or gulp launch over the group's sh.rows rows (row0:
// the tensors' first rows, row0[n] = sh.rows): up to max_per_cu workgroups
// per CU where their LDS fits, else fewer (M = 8's registers allow only
// one); T rows per workgroup (quad mode: a multiple of four); the fewest
// column phases P (a divisor of NB) whose activation slice fits in LDS;
// within a phase, the segments that give the fewest block-times per
// workgroup (a unit's closing sum and cursor step, per activation row,
// costing `unit_cost` of a block: unit_end_cost()). W is the kernel's waves
// per workgroup, quad whether
// its verify rows run in quad units, `fixed` its static LDS; a second
// exponent table is added when a tile spans two tensors (allowed only with
// `allow_two`). Without it, a group whose tensor boundaries the even tile
// would cut takes the tile height, from T/2 to 4T, that divides every
// boundary and puts the fewest rows on the busiest CU (the workgroups beyond
// the resident ones run as a later round). Returns false, planning nothing,
// when no plan fits.
inline bool plan_launch(SipShape& sh, const uint32_t* row0, uint32_t n, uint32_t min_rows, uint32_t M, uint32_t W,
                        uint32_t max_per_cu, bool quad, double unit_cost, size_t fixed, bool allow_two, uint32_t cus,
                        uint32_t& grid_out, size_t& lds_out, bool& two_out) {
    for (uint32_t per_cu = M == 8 ? 1 : max_per_cu; per_cu >= 1; --per_cu) {
        uint32_t grid = std::min<uint32_t>(sh.rows, cus * per_cu);
        uint32_t T = (sh.rows + grid - 1) / grid;
        if (quad) T = (T + 3) & ~3u;
        bool two = false;
        for (uint32_t i = 1; i < n; ++i) two |= row0[i] % T != 0;
        if (two && !allow_two) {
            uint32_t gb = 0;  // the tile height must divide every boundary
            for (uint32_t i = 1; i < n; ++i) gb = std::gcd(gb, row0[i]);
            uint32_t best = 0;
            uint64_t best_rows = ~0ull;
            for (uint32_t t = std::max(1u, T / 2); t <= 4 * T && t <= gb; ++t) {
                if (gb % t || (quad && t % 4)) continue;
                const uint64_t busiest = ((uint64_t)(sh.rows + t - 1) / t + cus - 1) / cus * t;
                if (busiest < best_rows || (busiest == best_rows && t > best)) {
                    best_rows = busiest;
                    best = t;
                }
            }
            if (best) {
                T = best;
                two = false;
            }
        }
        grid = (sh.rows + T - 1) / T;
        const uint32_t urows = quad ? (T + 3) / 4 : T;
        const uint32_t ublocks = quad ? 4 : 1;
        if (T <= min_rows && (allow_two || !two)) {
            for (uint32_t P = 1; P <= sh.nb; ++P) {
                if (sh.nb % P) continue;
                if (P > 1 && M >= 4 && per_cu > 1) {
                    // phased kernels at M >= 4 keep one workgroup per CU
                    // (quad and M = 8: their registers), unless one per CU
                    // would need phases too (gulp's v_dot2 rows: its
                    // phased kernel fits six waves per SIMD, and two
                    // workgroups per CU hide its decode better than one
                    // without phases; where one fits unphased, the phase
                    // barriers cost more than the second workgroup gains)
                    const size_t unphased = 2 * (size_t)M * (sh.nb * 1024) + fixed;
                    if (quad || M == 8 || unphased <= kLdsBytes) break;
                }
                const uint32_t K = sh.nb / P;
                double best = 1e30;
                uint32_t ps = 1;
                for (uint32_t s = 1; s <= std::min<uint32_t>(K, W); ++s) {
                    if (K % s) continue;
                    const double rounds = std::ceil((double)urows * s / W);
                    const double cost = P * rounds * ((double)ublocks * (K / s) + unit_cost * M);
                    if (cost < best - 1e-9) {
                        best = cost;
                        ps = s;
                    }
                }
                if (two && P > 1) break;  // (a tile spanning two tensors keeps every activation column resident)
                // the activation rows' stride: whole 1024-column blocks, plus
                // 16 bytes for the quad path's 16-byte operand reads (four
                // rows on distinct banks)
                const uint32_t xrow = K * 1024 + (quad ? 8 : 0);
                const size_t head = 2 * (size_t)M * xrow + (((size_t)T * P * ps * M * 4 + 15) & ~(size_t)15);
                const size_t lds = head + (two ? kTableBytes : 0);
                if ((lds + fixed) * per_cu > kLdsBytes) continue;
                sh.rows_per_wg = T;
                sh.phases = P;
                sh.phase_blocks = K;
                sh.xrow = xrow;
                sh.waves = W;
                sh.psegs = ps;
                sh.quad = quad;
                sh.segs = P * ps;
                sh.seg_blocks = K / ps;
                const uint32_t pu = urows * ps, rem = W % pu;
                sh.dp = W / pu;
                sh.dr = rem / ps;
                sh.ds = rem - sh.dr * ps;
                sh.tbl2_lds = two ? (uint32_t)head : 0u;
                // the dispatcher gives each CU one of the first cus
                // workgroups, then a second from the rest; past 2 cus (a
                // tile height that divides the group's boundaries) the
                // later workgroups are no CU's second, only a later round,
                // and the raised priority would take issue slots from the
                // running ones (Qwen3-8B q/k/v at M = 4 7% slower with it,
                // the 32B-class 26%), so no workgroup gets it
                sh.young_from = per_cu == 2 && grid <= 2 * cus ? cus : ~0u;
                grid_out = grid;
                lds_out = lds;
                two_out = two;
                return true;
            }
        }
        if (per_cu == 1) break;
    }
    return false;
}

// gulp's launch plan. A group whose tensor boundaries the tiles must not
// cut can take more tiles than two workgroups per CU hold: its later tiles
// then run as another round, and tiles of few rows leave waves of a
// 12-wave workgroup without a unit. Those launches (more than two tiles a
// CU, at most three) run 8-wave workgroups, three per CU, all resident at
// once.
inline bool plan_gulp(SipShape& sh, const uint32_t* row0, uint32_t n, uint32_t min_rows, uint32_t M, uint32_t cus,
                      uint32_t& grid_out, size_t& lds_out, bool& two_out, bool matrix = false) {
    const bool quad = gulp_quad((int)M, matrix);
    const double uc = unit_end_cost(true, (int)M, false, matrix);
    if (!plan_launch(sh, row0, n, min_rows, M, kPlanWaves, gulp_per_cu((int)M, matrix), quad, uc, kGulpStaticLds,
                     false, cus, grid_out, lds_out, two_out))
        return false;
    if (!quad && grid_out > 2 * cus && grid_out <= 3 * cus) {
        SipShape s3 = sh;
        uint32_t g3 = 0;
        size_t l3 = 0;
        bool t3 = false;
        if (plan_launch(s3, row0, n, min_rows, M, kGulpWaves3, 3, false, uc, kGulpStaticLds, false, cus, g3, l3, t3) &&
            g3 <= 3 * cus && s3.phases == 1 && (l3 + kGulpStaticLds) * 3 <= kLdsBytes) {
            sh = s3;
            grid_out = g3;
            lds_out = l3;
            two_out = t3;
        }
    }
    return true;
}

}  // namespace dmx
