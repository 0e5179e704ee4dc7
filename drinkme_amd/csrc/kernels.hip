// Device half of libdmx_radix.so: gfx950 (CDNA4) kernels for drinkme's
// radix-coded bf16 weights and the C-ABI entry points that launch them.
//
//   k_decode          every block to its u16 bit patterns
//                     (radix_ops.decode_bits, radix_kernel_gpu.py:614-636)
//   k_schedule        the per-block tier stream lengths
//                     (radix_ops.prepare_schedule, radix_kernel_gpu.py:44-66)
//   k_gemv_generic    decode + GEMV for any widths, block size, ragged rows,
//                     M = 1..8 (radix_ops.gemv_fused / gemv_mc,
//                     radix_kernel_gpu.py:682-718, radix_ops.py:91-164)
//   k_gemv_sip        the M = 1 fused decode + GEMV for sip (3, 8) streams
//                     over whole 1024-weight blocks and a bf16 activation —
//                     the serial decode step's hot kernel
//
// Bit layout (src/drinkme/codec/radix.py:77-136): per block of n weights,
// the 8-bit literal plane (sign << 7 | mantissa), then per nonterminal tier
// one w-bit code per weight still unresolved, in order, code = min(rank -
// base, 2^w - 1), then the raw 8-bit exponents of the weights no tier
// resolved; every stream zero-padded to whole u32 words, fields
// little-endian. Weight bits = (lit & 0x7F) | (lit >> 7) << 15 | exp << 7.
//
// No kernel bounds-checks its payload reads: with a directory that passed
// the descriptor gate, every read lies within block_word_bounds(B)[1] words
// of the block's start, inside the zero pad the caller allocates after the
// payload (src/drinkme/codec/swap.py:84-95).
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <cmath>

#include "dmx_radix.h"

namespace {

constexpr int kWave = 64;

// ---------------------------------------------------------------- helpers --

struct Desc {
    const uint32_t* data;
    const uint32_t* offsets;
    const uint8_t* table;  // the padded per-tier palette tables, as bytes
    uint32_t rows, cols, block, nb, tiers;
    uint32_t width[8];
    uint32_t table_byte[8];  // byte offset of tier j's table
};

__device__ __forceinline__ uint32_t words_for(uint32_t count, uint32_t width) { return (count * width + 31u) >> 5; }

// Field i of width w (<= 8) of the little-endian stream at s.
__device__ __forceinline__ uint32_t field(const uint32_t* s, uint32_t i, uint32_t w) {
    uint32_t bit = i * w, sh = bit & 31u;
    const uint32_t* p = s + (bit >> 5);
    uint32_t v = p[0] >> sh;
    if (sh + w > 32u) v |= p[1] << (32u - sh);
    return v & ((1u << w) - 1u);
}

__device__ __forceinline__ uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
__device__ __forceinline__ uint32_t lane_id() { return threadIdx.x & 63u; }

// Inclusive prefix sum over the 64 lanes: row_shr 1, 2, 4, 8 inside each
// 16-lane row, then row_bcast 15 / 31 carry the rows' totals forward.
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
    v += __builtin_amdgcn_update_dpp(0u, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0u, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0u, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0u, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0u, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0u, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Sum over the 64 lanes (a fixed tree: deterministic).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
    return v;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float load_elem(const void* p, int dtype, uint64_t i) {
    return dtype == DMX_BF16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_elem(void* p, int dtype, uint64_t i, float v) {
    if (dtype == DMX_BF16)
        static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(v);
    else
        static_cast<float*>(p)[i] = v;
}

// ------------------------------------------------- the generic block decoder --
//
// One workgroup of kGenThreads decodes one block: thread t owns the K
// consecutive weights t*K .. t*K + K - 1 (K = max(1, B / 256), at most 16).
// Per tier, each still-unresolved weight's slot in the tier's stream is its
// rank among the unresolved weights: a workgroup exclusive scan of the
// threads' counts plus the thread's own running count.

constexpr int kGenThreads = 256;
constexpr int kGenWaves = kGenThreads / kWave;
constexpr int kGenK = 16;

// Exclusive prefix of v over the workgroup; `total` = the sum. `sh` holds
// kGenWaves words of LDS and is reusable when this returns.
__device__ __forceinline__ uint32_t wg_scan_excl(uint32_t v, uint32_t* sh, uint32_t& total) {
    uint32_t inc = wave_scan_incl(v);
    uint32_t w = threadIdx.x >> 6;
    if (lane_id() == 63) sh[w] = inc;
    __syncthreads();
    uint32_t before = 0, tot = 0;
#pragma unroll
    for (int k = 0; k < kGenWaves; ++k) {
        uint32_t s = sh[k];
        before += (uint32_t)k < w ? s : 0u;
        tot += s;
    }
    __syncthreads();
    total = tot;
    return before + inc - v;
}

// Decodes block `blk` (n weights) into bits[k] for k < K; weights past n
// come back 0. When `counts` is non-null, thread 0 also receives each
// tier's entry count (tier j: counts[j]; the terminal: counts[tiers - 1]).
__device__ void decode_block(const Desc& d, uint32_t blk, uint32_t n, uint32_t K, uint32_t (&bits)[kGenK],
                             uint32_t* sh, uint32_t* counts) {
    const uint32_t t = threadIdx.x;
    const uint32_t start = d.offsets[blk], end = d.offsets[blk + 1];
    const uint8_t* lit = reinterpret_cast<const uint8_t*>(d.data + start);
    uint32_t active = 0;
#pragma unroll
    for (int k = 0; k < kGenK; ++k) {
        uint32_t i = t * K + k;
        bits[k] = 0;
        if ((uint32_t)k < K && i < n) {
            uint32_t l = lit[i];
            bits[k] = (l & 0x7Fu) | ((l >> 7) << 15);
            active |= 1u << k;
        }
    }
    uint32_t pos = start + words_for(n, 8);
    for (uint32_t level = 0; level + 1 < d.tiers; ++level) {
        const uint32_t w = d.width[level], esc = (1u << w) - 1u;
        const uint8_t* tab = d.table + d.table_byte[level];
        uint32_t count;
        uint32_t r = wg_scan_excl(__builtin_popcount(active), sh, count);
        if (counts && t == 0) counts[level] = count;
        const uint32_t* s = d.data + pos;
#pragma unroll
        for (int k = 0; k < kGenK; ++k) {
            if (active & (1u << k)) {
                uint32_t code = field(s, r++, w);
                if (code != esc) {
                    if (d.table) bits[k] |= (uint32_t)tab[code] << 7;
                    active &= ~(1u << k);
                }
            }
        }
        pos += words_for(count, w);
    }
    uint32_t count;
    uint32_t r = wg_scan_excl(__builtin_popcount(active), sh, count);
    if (counts && t == 0) counts[d.tiers - 1] = count;
    // the terminal stream is read only where the directory gives the block
    // words past its nonterminal streams (radix_kernel_gpu.py:96-98)
    if (end > pos) {
        const uint32_t* s = d.data + pos;
#pragma unroll
        for (int k = 0; k < kGenK; ++k)
            if (active & (1u << k)) bits[k] |= field(s, r++, 8) << 7;
    }
}

__global__ __launch_bounds__(kGenThreads) void k_decode(Desc d, uint16_t* __restrict__ out) {
    __shared__ uint32_t sh[kGenWaves];
    const uint32_t blk = blockIdx.x, row = blk / d.nb, b = blk % d.nb;
    const uint32_t c0 = b * d.block, n = min(d.block, d.cols - c0);
    const uint32_t K = d.block > (uint32_t)kGenThreads ? d.block / kGenThreads : 1u;
    uint32_t bits[kGenK];
    decode_block(d, blk, n, K, bits, sh, nullptr);
    uint16_t* dst = out + (uint64_t)row * d.cols + c0;
#pragma unroll
    for (int k = 0; k < kGenK; ++k) {
        uint32_t i = threadIdx.x * K + k;
        if ((uint32_t)k < K && i < n) dst[i] = (uint16_t)bits[k];
    }
}

__global__ __launch_bounds__(kGenThreads) void k_schedule(Desc d, uint16_t* __restrict__ sched) {
    __shared__ uint32_t sh[kGenWaves];
    __shared__ uint32_t counts[8];
    const uint32_t blk = blockIdx.x, b = blk % d.nb;
    const uint32_t n = min(d.block, d.cols - b * d.block);
    const uint32_t K = d.block > (uint32_t)kGenThreads ? d.block / kGenThreads : 1u;
    uint32_t bits[kGenK];
    decode_block(d, blk, n, K, bits, sh, counts);
    if (threadIdx.x == 0) {
        uint32_t header = 0;
        for (uint32_t level = 1; level + 1 < d.tiers; ++level)
            header |= words_for(counts[level], d.width[level]) << ((level - 1) * 8);
        sched[blk] = (uint16_t)header;
    }
}

// One workgroup per output row: the row's blocks decoded in turn, each
// weight multiplied into M fp32 accumulators; the row's sums reduced over
// the workgroup in a fixed order, the bias added in fp32, one rounding.
template <int M>
__global__ __launch_bounds__(kGenThreads) void k_gemv_generic(Desc d, const void* __restrict__ x, int x_dtype,
                                                              const void* __restrict__ bias, int bias_dtype,
                                                              void* __restrict__ out, int out_dtype) {
    __shared__ uint32_t sh[kGenWaves];
    __shared__ float red[M][kGenWaves];
    const uint32_t row = blockIdx.x;
    const uint32_t K = d.block > (uint32_t)kGenThreads ? d.block / kGenThreads : 1u;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    for (uint32_t b = 0; b < d.nb; ++b) {
        const uint32_t c0 = b * d.block, n = min(d.block, d.cols - c0);
        uint32_t bits[kGenK];
        decode_block(d, row * d.nb + b, n, K, bits, sh, nullptr);
#pragma unroll
        for (int k = 0; k < kGenK; ++k) {
            uint32_t i = threadIdx.x * K + k;
            if ((uint32_t)k < K && i < n) {
                float w = bf16_bits_to_f32(bits[k]);
#pragma unroll
                for (int m = 0; m < M; ++m) acc[m] = fmaf(w, load_elem(x, x_dtype, (uint64_t)m * d.cols + c0 + i), acc[m]);
            }
        }
    }
    const uint32_t wv = threadIdx.x >> 6;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float s = wave_sum(acc[m]);
        if (lane_id() == 0) red[m][wv] = s;
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)M) {
        const int m = threadIdx.x;
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < kGenWaves; ++k) s += red[m][k];
        if (bias) s += load_elem(bias, bias_dtype, row);
        store_elem(out, out_dtype, (uint64_t)m * d.rows + row, s);
    }
}

// ------------------------------------------------- sip, M = 1, whole blocks --
//
// Work split: one resident workgroup of kSipWaves waves per slot (two per
// CU). Workgroup g owns rows [g T, g T + T); each row is cut into S equal
// segments of L = NB / S blocks, and the T * S (row, segment) units are
// dealt to the waves round-robin, so every wave gets the same number of
// blocks (T, S chosen on the host for that). Unit u covers the workgroup's
// blocks [u L, u L + L) in row-major order. Each wave streams its blocks with
// two blocks of loads in flight, sums a unit over its lanes and parks it in
// LDS; one barrier at the end, then each row's S partials are added in
// segment order, the bias added, one rounding.
//
// Within a block, lane l owns weights 16l .. 16l + 15: its literals are the
// 16 bytes at word 4l (one 128-bit load) and its sixteen 3-bit tier-0 codes
// the 48 bits at bit 48l of the tier-0 stream (two words). Per group of four
// weights, a 4096-entry LDS table indexed by their four codes gives the
// exponent fields of the group's two bf16 pairs — E(c) << 7 | E(c') << 23,
// with E of the escape code (7) = 0 — and, in bits 3..6 of the first word,
// the group's escape flags m. A pair is then one byte-permute of the
// literals merged (v_bfi) with its table word, and one v_dot2_f32_bf16 with
// the activation pair from LDS.
//
// Escapes are patched into the exponent words before the products, so every
// weight is its exact bf16 value. A group's escapes are terminal bytes
// q .. q + popcount(m) - 1, where q is the wave's exclusive prefix of
// per-lane escape counts (one DPP scan) plus the lane's earlier groups: the
// four bytes from q come out of the wave's LDS copy of the terminal stream
// with one funnel shift, and a 16-entry selector table indexed by m places
// byte r (the r-th escape of the group) in its pair's exponent field.

constexpr int kSipWaves = 12;
constexpr int kSipThreads = kSipWaves * kWave;
constexpr uint32_t kSipFixed = 256 + 96;  // literal plane + tier 0 words of a 1024-weight block
constexpr uint32_t kTableBytes = 4096 * 8;
constexpr uint32_t kSelBytes = (16 + 9 * 16) * 8;
constexpr uint32_t kTermWords = 264;  // the widest terminal (256 words) + a window's overhang, per wave

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_ptr;
typedef __attribute__((address_space(1))) void* glb_ptr;

__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc,
                                           false);
}

// Sum over the 64 lanes as an inclusive DPP scan (fixed order); lane 63's
// value, broadcast.
__device__ __forceinline__ float wave_sum_dpp(float v) {
#define DMX_DPP_ADD(ctrl, rmask) \
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rmask, 0xF, false))
    DMX_DPP_ADD(0x111, 0xF);
    DMX_DPP_ADD(0x112, 0xF);
    DMX_DPP_ADD(0x114, 0xF);
    DMX_DPP_ADD(0x118, 0xF);
    DMX_DPP_ADD(0x142, 0xA);
    DMX_DPP_ADD(0x143, 0xC);
#undef DMX_DPP_ADD
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

struct SipShape {
    uint32_t rows, cols, nb;
    uint32_t rows_per_wg;  // T
    uint32_t segs;         // S
    uint32_t seg_blocks;   // L = NB / S
    int bias_dtype, out_dtype;
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct SipStage {
    u32x4 lit;
    u32x2 t0;
    uint32_t term;
    uint32_t start, end;
};

// A block's directory pair, read through the scalar cache.
__device__ __forceinline__ uint2 sip_offsets(const uint32_t* __restrict__ offsets, uint32_t blk) {
    uint2 o;
    __builtin_memcpy(&o, offsets + blk, 8);
    return o;
}

// Per-lane byte offsets of a block's loads: the lane's 16 literal bytes, its
// two tier-0 words (48 bits at bit 48l) and word l of the terminal region.
struct SipLanes {
    uint32_t lit, t0, term;
};

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// A raw buffer resource over [base, base + bytes): 32-bit dword format, no
// stride, the range checked against `bytes`.
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4 r;
    r.x = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(a >> 32) & 0xFFFF);
    r.z = (int32_t)bytes;
    r.w = 0x00020000;
    return r;
}

// A block's loads through the workgroup's buffer resource (based at the
// workgroup's first block, so every byte offset is small): the terminal
// word, the tier-0 pair and the literals, issued as one unit of three
// vector loads. They are written as instructions the compiler does not
// track, so the only waits on them are the explicit SIP_WAIT below, placed
// where a stage is consumed: loads return in issue order, so waiting until
// at most N newer loads are outstanding completes the stage, whatever other
// loads the compiler adds after it. Every read lies within the block's
// start + 352 + 64 words, inside block_word_bounds(1024)[1] = 608.
__device__ __forceinline__ SipStage sip_load(i32x4 rsrc, uint32_t wg_start, uint2 o, const SipLanes& ln) {
    SipStage s;
    s.start = o.x;
    s.end = o.y;
    const uint32_t soff = (o.x - wg_start) * 4u;
    asm volatile(
        "buffer_load_dword %0, %3, %6, %7 offen\n\t"
        "buffer_load_dwordx2 %1, %4, %6, %7 offen\n\t"
        "buffer_load_dwordx4 %2, %5, %6, %7 offen"
        : "=&v"(s.term), "=&v"(s.t0), "=&v"(s.lit)
        : "v"(ln.term), "v"(ln.t0), "v"(ln.lit), "s"(rsrc), "s"(soff));
    return s;
}

// Completes stage S: at most N vector loads issued after it still in flight.
// The "+v" operands make S's registers this statement's results, so nothing
// reads them before the wait.
#define SIP_WAIT(N, S) asm volatile("s_waitcnt vmcnt(" #N ")" : "+v"(S.lit), "+v"(S.t0), "+v"(S.term))

// A wave's place in its work: unit u, block j of the unit, the block's
// global index and its column block.
struct SipCursor {
    uint32_t u, j, blk, cb;
};

__device__ __forceinline__ void sip_start(const SipShape& sh, SipCursor& c, uint32_t u, uint32_t r0) {
    c.u = u;
    c.j = 0;
    c.blk = r0 * sh.nb + u * sh.seg_blocks;
    c.cb = (u % sh.segs) * sh.seg_blocks;
}

__device__ __forceinline__ void sip_next(const SipShape& sh, SipCursor& c, uint32_t r0) {
    if (++c.j == sh.seg_blocks)
        sip_start(sh, c, c.u + kSipWaves, r0);
    else {
        ++c.blk;
        ++c.cb;
    }
}

__global__ __launch_bounds__(kSipThreads, 6) void k_gemv_sip(const uint32_t* __restrict__ data,
                                                          const uint32_t* __restrict__ offsets,
                                                          const uint32_t* __restrict__ palette,
                                                          const uint16_t* __restrict__ x, const void* __restrict__ bias,
                                                          void* __restrict__ out, SipShape sh) {
    // fixed-size tables in static LDS (their addresses fold into the LDS
    // instructions' offsets); the activation and the row partials after them
    __shared__ uint2 tbl[4096];
    __shared__ uint2 sel[16];
    __shared__ uint2 sel2[9 * 16];
    __shared__ uint32_t term_all[kSipWaves * kTermWords];
    extern __shared__ __align__(16) uint8_t lds_dyn[];
    uint16_t* xs = reinterpret_cast<uint16_t*>(lds_dyn);
    float* red = reinterpret_cast<float*>(lds_dyn + 2 * sh.cols);

    const uint32_t wv = wave_id(), lane = lane_id();
    const uint32_t r0 = blockIdx.x * sh.rows_per_wg;
    const uint32_t nrows = min(sh.rows - r0, sh.rows_per_wg);
    const uint32_t units = nrows * sh.segs;
    uint32_t* term = term_all + wv * kTermWords;

    // the activation goes to LDS by direct loads (no registers staged), first
    // in the queue: small and hot in L2; the barrier below waits for it
    const uint32_t xchunks = sh.cols / 8;
    for (uint32_t i = threadIdx.x; i < xchunks; i += kSipThreads)
        __builtin_amdgcn_global_load_lds((glb_ptr)(reinterpret_cast<const uint4*>(x) + i),
                                         (lds_ptr)(reinterpret_cast<uint4*>(xs) + (i - lane)), 16, 0, 0);

    // the first two blocks' loads go out before the tables are built; a
    // cursor past the wave's work reads the workgroup's first block instead
    const uint32_t first_blk = r0 * sh.nb;
    SipCursor p, c;
    sip_start(sh, p, wv, r0);
    c = p;
    // the workgroup's payload window: from its first block's first word
    const uint32_t wg_start = offsets[first_blk];
    const i32x4 rsrc = make_rsrc(data + wg_start, 0x7FFFFFFFu);
    SipLanes ln;
    ln.lit = 16 * lane;
    ln.t0 = 1024 + 4 * ((3 * lane) >> 1);
    ln.term = 4 * (kSipFixed + lane);
    auto next_offsets = [&]() {
        uint2 o = sip_offsets(offsets, p.u < units ? p.blk : first_blk);
        sip_next(sh, p, r0);
        return o;
    };
    const uint2 oA = next_offsets(), oB = next_offsets();
    uint2 oC = next_offsets();
    // the prologue's two stages issue in the loop's order (no interleaving),
    // so the waits the loop needs are the same on entry as in steady state
    SipStage sA = sip_load(rsrc, wg_start, oA, ln);
    __builtin_amdgcn_sched_barrier(0);
    SipStage sB = sip_load(rsrc, wg_start, oB, ln);
    __builtin_amdgcn_sched_barrier(0);
    SipStage sC;

    // the exponent table of this tensor's palette: byte c of the two table
    // words is E(c), byte 7 the zero pad the escape code reads
    const uint32_t p0 = palette[0], p1 = palette[1];
    for (uint32_t g = threadIdx.x; g < 4096; g += kSipThreads) {
        uint32_t c0 = g & 7, c1 = (g >> 3) & 7, c2 = (g >> 6) & 7, c3 = (g >> 9) & 7;
        uint32_t e0 = __builtin_amdgcn_perm(p1, p0, c0) & 0xFF, e1 = __builtin_amdgcn_perm(p1, p0, c1) & 0xFF;
        uint32_t e2 = __builtin_amdgcn_perm(p1, p0, c2) & 0xFF, e3 = __builtin_amdgcn_perm(p1, p0, c3) & 0xFF;
        uint32_t m = (c0 == 7) | ((c1 == 7) << 1) | ((c2 == 7) << 2) | ((c3 == 7) << 3);
        tbl[g] = make_uint2((e0 << 7) | (e1 << 23) | (m << 3), (e2 << 7) | (e3 << 23));
    }
    // selectors of escape mask m (4 weights) at offset o: byte 0 / 2 of word
    // k / 2 picks, for weight k of the group, the window byte of its escape
    // (o + its rank among the group's escapes), or 0x0C (a zero byte) when
    // k did not escape. sel: o = 0 (a window per group); sel2[o][m]: one
    // 8-byte window per lane, o = the lane's escapes in earlier groups.
    for (uint32_t i = threadIdx.x; i < 9 * 16; i += kSipThreads) {
        const uint32_t m = i & 15, o = i >> 4;
        uint32_t b[4];
        for (uint32_t k = 0, r = o; k < 4; ++k) b[k] = (m >> k) & 1 ? (r++ & 7) : 0x0Cu;
        const uint2 e = make_uint2(b[0] | 0x0C00u | (b[1] << 16) | 0x0C000000u,
                                   b[2] | 0x0C00u | (b[3] << 16) | 0x0C000000u);
        sel2[i] = e;
        if (o == 0) sel[m] = e;
    }
    // every wave's direct loads into LDS must land before any wave reads
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    const uint32_t keep = 0x807F807Fu;  // sign + mantissa bits of a bf16 pair, from the literal
    float acc0 = 0.0f, acc1 = 0.0f;
    // one block of the wave's work, from its loaded stage
    auto process = [&](const SipStage& s0) {
        const uint64_t v = ((uint64_t)s0.t0.y << 32 | s0.t0.x) >> ((lane & 1) * 16);
        const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
        uint2 E0 = tbl[lo & 0xFFF];
        uint2 E1 = tbl[(lo >> 12) & 0xFFF];
        uint2 E2 = tbl[__builtin_amdgcn_alignbit(hi, lo, 24) & 0xFFF];
        uint2 E3 = tbl[(hi >> 4) & 0xFFF];
        const uint16_t* xb = xs + c.cb * 1024 + 16 * lane;
        uint4 xa, xc;
        __builtin_memcpy(&xa, xb, 16);
        __builtin_memcpy(&xc, xb + 8, 16);

        // escapes: group g's flags are bits 3..6 of E_g.x (a_g = m_g << 3);
        // a lane's escapes are terminal bytes q0 .. q0 + cnt - 1
        const uint32_t a0 = E0.x & 0x78u, a1 = E1.x & 0x78u, a2 = E2.x & 0x78u, a3 = E3.x & 0x78u;
        const uint32_t q1_ = __builtin_popcount(a0), q2_ = q1_ + __builtin_popcount(a1);
        const uint32_t q3_ = q2_ + __builtin_popcount(a2), cnt = q3_ + __builtin_popcount(a3);
        const uint32_t q0 = wave_scan_incl(cnt) - cnt;
        // the terminal is read only when the directory gives the block words
        // past its fixed streams (radix_kernel_gpu.py:96-98); without it the
        // escaped exponents stay 0
        const bool has_term = s0.end > s0.start + kSipFixed;
        const uint32_t tw = has_term ? s0.term : 0u;  // lane j: terminal word j
        // common case: every lane's escapes (at most 8) lie in words 0..62
        if (__builtin_amdgcn_ballot_w64(cnt > 8 || q0 > 243) == 0) {
            const int k0 = (int)(q0 & ~3u);
            const uint32_t w0 = __builtin_amdgcn_ds_bpermute(k0, tw);
            const uint32_t w1 = __builtin_amdgcn_ds_bpermute(k0 + 4, tw);
            const uint32_t w2 = __builtin_amdgcn_ds_bpermute(k0 + 8, tw);
            const uint32_t wlo = __builtin_amdgcn_alignbit(w1, w0, q0 << 3);
            const uint32_t whi = __builtin_amdgcn_alignbit(w2, w1, q0 << 3);
#define DMX_PATCH2(E, a, off)                                                   \
    {                                                                           \
        const uint2 s = sel2[((off) << 4) | ((a) >> 3)];                        \
        E.x |= __builtin_amdgcn_perm(whi, wlo, s.x) << 7;                       \
        E.y |= __builtin_amdgcn_perm(whi, wlo, s.y) << 7;                       \
    }
            DMX_PATCH2(E0, a0, 0)
            DMX_PATCH2(E1, a1, q1_)
            DMX_PATCH2(E2, a2, q2_)
            DMX_PATCH2(E3, a3, q3_)
#undef DMX_PATCH2
        } else if (has_term) {
            // a lane with more than 8 escapes, or more than 243 before it: the
            // terminal staged in the wave's LDS slot, a window per group
            const uint32_t total = __builtin_amdgcn_readlane(q0 + cnt, 63);
            term[lane] = tw;
            for (uint32_t k = lane + kWave; k < ((total + 3) >> 2) + 2; k += kWave)
                term[k] = data[s0.start + kSipFixed + k];
            __builtin_amdgcn_wave_barrier();
#define DMX_PATCH(E, a, qoff)                                                   \
    {                                                                           \
        const uint32_t q = q0 + (qoff);                                         \
        const uint2 s = sel[(a) >> 3];                                          \
        const uint32_t* wp = term + (q >> 2);                                   \
        const uint32_t w = __builtin_amdgcn_alignbit(wp[1], wp[0], q << 3);     \
        E.x |= __builtin_amdgcn_perm(0u, w, s.x) << 7;                          \
        E.y |= __builtin_amdgcn_perm(0u, w, s.y) << 7;                          \
    }
            DMX_PATCH(E0, a0, 0)
            DMX_PATCH(E1, a1, q1_)
            DMX_PATCH(E2, a2, q2_)
            DMX_PATCH(E3, a3, q3_)
#undef DMX_PATCH
            __builtin_amdgcn_wave_barrier();
        }
        const uint32_t L0 = s0.lit.x, L1 = s0.lit.y, L2 = s0.lit.z, L3 = s0.lit.w;
        acc0 = dot2((__builtin_amdgcn_perm(L0, L0, 0x01010000) & keep) | (E0.x & ~keep), xa.x, acc0);
        acc1 = dot2((__builtin_amdgcn_perm(L0, L0, 0x03030202) & keep) | (E0.y & ~keep), xa.y, acc1);
        acc0 = dot2((__builtin_amdgcn_perm(L1, L1, 0x01010000) & keep) | (E1.x & ~keep), xa.z, acc0);
        acc1 = dot2((__builtin_amdgcn_perm(L1, L1, 0x03030202) & keep) | (E1.y & ~keep), xa.w, acc1);
        acc0 = dot2((__builtin_amdgcn_perm(L2, L2, 0x01010000) & keep) | (E2.x & ~keep), xc.x, acc0);
        acc1 = dot2((__builtin_amdgcn_perm(L2, L2, 0x03030202) & keep) | (E2.y & ~keep), xc.y, acc1);
        acc0 = dot2((__builtin_amdgcn_perm(L3, L3, 0x01010000) & keep) | (E3.x & ~keep), xc.z, acc0);
        acc1 = dot2((__builtin_amdgcn_perm(L3, L3, 0x03030202) & keep) | (E3.y & ~keep), xc.w, acc1);

        if (c.j + 1 == sh.seg_blocks) {
            const float s = wave_sum_dpp(acc0 + acc1);
            if (lane == 0) red[c.u] = s;
            acc0 = acc1 = 0.0f;
        }
        sip_next(sh, c, r0);
    };
    // three stages rotate roles (no register copies); each step issues the
    // stage two blocks ahead, then completes the oldest (six loads newer);
    // whole rounds of three blocks, then the remainder
    const uint32_t my_units = wv < units ? (units - wv + kSipWaves - 1) / kSipWaves : 0;
    const uint32_t items = my_units * sh.seg_blocks;
    uint32_t k = 0;
    for (; k + 3 <= items; k += 3) {
        sC = sip_load(rsrc, wg_start, oC, ln);
        uint2 oN = next_offsets();
        SIP_WAIT(6, sA);
        process(sA);
        sA = sip_load(rsrc, wg_start, oN, ln);
        oN = next_offsets();
        SIP_WAIT(6, sB);
        process(sB);
        sB = sip_load(rsrc, wg_start, oN, ln);
        oC = next_offsets();
        SIP_WAIT(6, sC);
        process(sC);
    }
    // in flight now: sA (older), then sB
    SIP_WAIT(3, sA);
    if (k < items) process(sA);
    SIP_WAIT(0, sB);
    if (k + 1 < items) process(sB);
    __syncthreads();
    for (uint32_t t = threadIdx.x; t < nrows; t += kSipThreads) {
        float sum = 0.0f;
        for (uint32_t k = 0; k < sh.segs; ++k) sum += red[t * sh.segs + k];
        if (bias) sum += load_elem(bias, sh.bias_dtype, r0 + t);
        store_elem(out, sh.out_dtype, r0 + t, sum);
    }
}

// ------------------------------------------------------------- host side --

int fail(char* err, size_t n, const char* msg) {
    if (err && n) {
        strncpy(err, msg, n - 1);
        err[n - 1] = 0;
    }
    return 1;
}

int fail_hip(char* err, size_t n, const char* what, hipError_t e) {
    char buf[256];
    snprintf(buf, sizeof buf, "%s: %s", what, hipGetErrorString(e));
    return fail(err, n, buf);
}

std::atomic<int> g_policy{DMX_POLICY_AUTO};

uint64_t pad_words_for(uint32_t block, const uint32_t* w, uint32_t nw) {
    if (nw < 2 || nw > 8 || w[nw - 1] != 8) return 0;
    uint64_t most = (uint64_t(block) * 8 + 31) / 32;
    for (uint32_t j = 0; j < nw; ++j) {
        if (w[j] < 1 || w[j] > 8) return 0;
        most += (uint64_t(block) * w[j] + 31) / 32;
    }
    return most;
}

// Host-side descriptor checks; fills the kernels' Desc.
int check_tensor(const dmx_radix_tensor* t, Desc& d, char* err, size_t errn, bool need_palette = true) {
    if (!t) return fail(err, errn, "null tensor descriptor");
    if (!t->data || !t->offsets || (need_palette && !t->palette))
        return fail(err, errn, "null device pointer in the tensor descriptor");
    if (t->rows == 0 || t->cols == 0) return fail(err, errn, "empty tensor");
    const uint32_t B = t->block_size;
    if (B < 32 || B > 4096 || (B & (B - 1))) return fail(err, errn, "block_size must be a power of two from 32 through 4096");
    if (t->n_widths < 2 || t->n_widths > 8 || t->widths[t->n_widths - 1] != 8)
        return fail(err, errn, "radix needs 2..8 widths in 1..8, ending with the exponent width");
    uint32_t covered = 0, table = 0;
    for (uint32_t j = 0; j < t->n_widths; ++j) {
        if (t->widths[j] < 1 || t->widths[j] > 8)
            return fail(err, errn, "radix needs 2..8 widths in 1..8, ending with the exponent width");
        d.width[j] = t->widths[j];
        if (j + 1 < t->n_widths) {
            d.table_byte[j] = table;
            covered += (1u << t->widths[j]) - 1;
            table += 4 * (((1u << t->widths[j]) + 2) / 4);
        }
    }
    if (covered > 256) return fail(err, errn, "radix tiers exceed the exponent alphabet");
    if (t->pad_words < pad_words_for(B, t->widths, t->n_widths))
        return fail(err, errn, "the payload needs block_word_bounds(B)[1] zero words of reach pad after it");
    if ((uint64_t)t->rows * ((t->cols + B - 1) / B) >= (1ull << 31)) return fail(err, errn, "too many blocks");
    d.data = t->data;
    d.offsets = t->offsets;
    d.table = reinterpret_cast<const uint8_t*>(t->palette);
    d.rows = t->rows;
    d.cols = t->cols;
    d.block = B;
    d.nb = (t->cols + B - 1) / B;
    d.tiers = t->n_widths;
    return 0;
}

int launch_check(char* err, size_t errn, const char* what) {
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : fail_hip(err, errn, what, e);
}

bool is_sip(const dmx_radix_tensor* t) { return t->n_widths == 2 && t->widths[0] == 3 && t->widths[1] == 8; }

int cu_count() {
    static std::atomic<int> cached{0};
    int n = cached.load();
    if (n) return n;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached.store(n);
    return n;
}

int launch_sip(const dmx_radix_tensor* t, const void* x, const void* bias, int bias_dtype, void* out, int out_dtype,
               hipStream_t stream, char* err, size_t errn) {
    SipShape sh;
    sh.rows = t->rows;
    sh.cols = t->cols;
    sh.nb = t->cols / 1024;
    sh.bias_dtype = bias_dtype;
    sh.out_dtype = out_dtype;
    // one workgroup per slot (two per CU), T rows each; S segments per row
    // so that the T * S units deal evenly to the 16 waves
    uint32_t grid = std::min<uint32_t>(sh.rows, (uint32_t)cu_count() * 2);
    sh.rows_per_wg = (sh.rows + grid - 1) / grid;
    grid = (sh.rows + sh.rows_per_wg - 1) / sh.rows_per_wg;
    double best = -1.0;
    sh.segs = 1;
    for (uint32_t s = 1; s <= std::min<uint32_t>(sh.nb, kSipWaves); ++s) {
        if (sh.nb % s) continue;
        const double units = (double)sh.rows_per_wg * s;
        const double eff = (units / kSipWaves) / std::ceil(units / kSipWaves);
        if (eff > best + 1e-9) {
            best = eff;
            sh.segs = s;
        }
    }
    sh.seg_blocks = sh.nb / sh.segs;
    const size_t lds = 2 * (size_t)sh.cols + (size_t)sh.rows_per_wg * sh.segs * 4;
    const size_t fixed = kTableBytes + kSelBytes + kSipWaves * kTermWords * 4;
    if (lds + fixed > 160 * 1024)
        return fail(err, errn, "sip gemv: the row tile does not fit in LDS");
    static std::atomic<size_t> lds_opted{64 * 1024 - fixed};
    if (lds > lds_opted.load()) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv_sip),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail_hip(err, errn, "sip kernel LDS opt-in", e);
        lds_opted.store(lds);
    }
    hipLaunchKernelGGL(k_gemv_sip, dim3(grid), dim3(kSipThreads), lds, stream, t->data, t->offsets, t->palette,
                       static_cast<const uint16_t*>(x), bias, out, sh);
    return launch_check(err, errn, "sip gemv launch");
}

template <int M>
void launch_generic_m(const Desc& d, const void* x, int x_dtype, const void* bias, int bias_dtype, void* out,
                      int out_dtype, hipStream_t stream) {
    hipLaunchKernelGGL(k_gemv_generic<M>, dim3(d.rows), dim3(kGenThreads), 0, stream, d, x, x_dtype, bias, bias_dtype,
                       out, out_dtype);
}

}  // namespace

extern "C" int dmx_abi_version(void) { return DMX_ABI_VERSION; }

extern "C" uint64_t dmx_radix_pad_words(uint32_t block_size, const uint32_t* widths, uint32_t n_widths) {
    if (!widths) return 0;
    return pad_words_for(block_size, widths, n_widths);
}

extern "C" int dmx_radix_set_policy(int policy) {
    if (policy != DMX_POLICY_AUTO && policy != DMX_POLICY_GENERIC) return -1;
    return g_policy.exchange(policy);
}

extern "C" int dmx_radix_decode(const dmx_radix_tensor* t, uint16_t* out, void* stream, char* err, size_t errn) {
    Desc d;
    if (check_tensor(t, d, err, errn)) return 1;
    if (!out) return fail(err, errn, "null output");
    hipLaunchKernelGGL(k_decode, dim3(d.rows * d.nb), dim3(kGenThreads), 0, static_cast<hipStream_t>(stream), d, out);
    return launch_check(err, errn, "decode launch");
}

extern "C" int dmx_radix_prepare(const dmx_radix_tensor* t, uint16_t* schedule, void* stream, char* err, size_t errn) {
    Desc d;
    if (check_tensor(t, d, err, errn, false)) return 1;
    if (!schedule) return fail(err, errn, "null schedule output");
    if (t->n_widths <= 2) return fail(err, errn, "a two-tier profile has no schedule");
    hipLaunchKernelGGL(k_schedule, dim3(d.rows * d.nb), dim3(kGenThreads), 0, static_cast<hipStream_t>(stream), d,
                       schedule);
    return launch_check(err, errn, "schedule launch");
}

extern "C" int dmx_radix_gemv(const dmx_radix_tensor* t, const void* x, int x_dtype, uint32_t m, const void* bias,
                              int bias_dtype, void* out, int out_dtype, void* stream, char* err, size_t errn) {
    Desc d;
    if (check_tensor(t, d, err, errn)) return 1;
    if (!x || !out) return fail(err, errn, "null activation or output");
    if (m < 1 || m > 8) return fail(err, errn, "m outside 1..8");
    if ((x_dtype != DMX_BF16 && x_dtype != DMX_F32) || (out_dtype != DMX_BF16 && out_dtype != DMX_F32) ||
        (bias && bias_dtype != DMX_BF16 && bias_dtype != DMX_F32))
        return fail(err, errn, "dtype must be DMX_BF16 or DMX_F32");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    if (g_policy.load() == DMX_POLICY_AUTO && m == 1 && x_dtype == DMX_BF16 && is_sip(t) && t->block_size == 1024 &&
        t->cols % 1024 == 0 && aligned)
        return launch_sip(t, x, bias, bias_dtype, out, out_dtype, s, err, errn);
    switch (m) {
        case 1: launch_generic_m<1>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 2: launch_generic_m<2>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 3: launch_generic_m<3>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 4: launch_generic_m<4>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 5: launch_generic_m<5>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 6: launch_generic_m<6>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 7: launch_generic_m<7>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        default: launch_generic_m<8>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
    }
    return launch_check(err, errn, "generic gemv launch");
}
