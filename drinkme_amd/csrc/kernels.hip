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
//   k_gemv_sip        the fused decode + GEMV for sip (3, 8) streams over
//                     whole 1024-weight blocks and M = 1..8 bf16 activation
//                     rows (radix_kernel_gpu.py:682-718, radix_ops.py:91-164)
//                     — the serial decode step's hot kernel; M = 4 and 8 in
//                     quad units on the matrix cores. Its other modes: the
//                     raw twin (a raw bf16 weight through the same plan and
//                     sums, radix_kernel_gpu.py:639-668) and the decode
//                     (each block's bits stored instead of the products)
//   k_gemv_gulp       the same for gulp (2, 2, 4, 8) streams
//                     (radix_kernel_gpu.py:292-392); M = 8 in quad units; a
//                     decode mode
//   k_gemv_narrow     a raw row-major bf16 weight against M <= 8 rows
//                     (radix_ops.gemv_narrow, radix_ops.py:177-249)
//
// The launch plan and the cursors that walk it are plan.h, shared with a
// host model of the kernels' reads.
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
#include <map>
#include <mutex>
#include <cmath>
#include <numeric>

#include "dmx_radix.h"
#include "plan.h"

namespace {

using namespace dmx;

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

// The same scan as six fused v_add_u32_dpp, written out: where the compiler
// keeps the zero of update_dpp in a register it no longer fuses the adds
// (twelve instructions and six register copies instead of six). A disabled
// row is not written, which adds 0; an out-of-row source reads 0
// (bound_ctrl). Two wait states before each DPP read of a VGPR written by
// the VALU just before it, and after the last write.
__device__ __forceinline__ uint32_t wave_scan_incl_dpp(uint32_t v) {
    asm volatile(
        "s_nop 1\n\t"
        "v_add_u32_dpp %0, %0, %0 row_shr:1 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_add_u32_dpp %0, %0, %0 row_shr:2 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_add_u32_dpp %0, %0, %0 row_shr:4 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_add_u32_dpp %0, %0, %0 row_shr:8 row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
        "s_nop 1\n\t"
        "v_add_u32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_add_u32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
        "s_nop 1"
        : "+v"(v));
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
// RAW: the raw twin, the row-major bf16 weight at d.data read at the
// positions the decode fills, everything else the same.
template <int M, bool RAW = false>
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
        if constexpr (RAW) {
            const uint16_t* wr = reinterpret_cast<const uint16_t*>(d.data) + (uint64_t)row * d.cols + c0;
#pragma unroll
            for (int k = 0; k < kGenK; ++k) {
                const uint32_t i = threadIdx.x * K + k;
                bits[k] = (uint32_t)k < K && i < n ? wr[i] : 0u;
            }
        } else {
            decode_block(d, row * d.nb + b, n, K, bits, sh, nullptr);
        }
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
// per-lane escape counts (one DPP scan) plus the lane's earlier groups. Lane
// j holds terminal word j; when every lane has at most 8 escapes, all below
// byte 252, a lane pulls its 12-byte window of the terminal with three
// cross-lane reads (ds_bpermute) and two funnel shifts, and a selector table
// indexed by (escapes before the group, m) places byte r (the r-th escape
// of the group) in its pair's exponent field. Otherwise (dense escapes, not
// seen in trained weights) each group's four bytes are read from memory.

constexpr int kSipWaves = (int)kPlanWaves;
constexpr int kSipThreads = kSipWaves * kWave;
// The sip kernel's progress balance (below): a margin of 12 measured best
// of 0, 6, 12, 24 and 48; on for launches of 12 or more blocks a wave (the
// Qwen3-8B step 1.9% faster than without, one layer 2.6%, 4096 x 4096
// GEMVs unchanged, which were 4-6% slower with it on).
constexpr uint32_t kBalanceMargin = 12, kBalanceMinBlocks = 12;

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

// Sum over each row of 16 lanes (inclusive DPP scan); lane 15 of the row
// holds it.
__device__ __forceinline__ float row_sum16(float v) {
#define DMX_DPP_ADD(ctrl) \
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, 0xF, 0xF, false))
    DMX_DPP_ADD(0x111);
    DMX_DPP_ADD(0x112);
    DMX_DPP_ADD(0x114);
    DMX_DPP_ADD(0x118);
#undef DMX_DPP_ADD
    return v;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Verify rows contracted four output rows at once (quad units). A wave
// decodes the blocks of rows 4q .. 4q + 3 at one column block in turn, each
// into its eight pair words h[j] (lane l: weights 16l .. 16l + 15 of row j),
// then transposes the four rows over the lanes of each quad so that lane
// 4b + i holds row i's weights 64b .. 64b + 63 (register set r: the 16
// weights lane 4b + r decoded). v_mfma_f32_4x4x4_16b_bf16 contracts 16
// independent 4 x 4 x 4 blocks; lane 4b + j of its result register i holds
// the sum over k < 4 of A[4b + i][k] B[4b + j][k] (its lane layout checked
// on gfx950 with integer operands). With A lane 4b + i = activation row i at
// columns 64b + 4s .. 64b + 4s + 3 and B lane 4b + j = output row j at the
// same columns, MFMA s (16 per block of four rows) keeps every product: lane
// 4b + j accumulates activation row i (register i) times output row j over
// its 64 columns, and a unit's end sums the 16 quads b.
typedef short bf16x4_t __attribute__((ext_vector_type(4)));

// The 4 x 4 transpose within each quad of lanes of four rows' pair words:
// after it, h[r][w] of lane 4b + i is the word w that lane 4b + r held for
// row i. Two butterfly stages, one per lane bit, each DPP reads of the
// partner lane and one blend per word. A blend is a byte permute with a
// per-lane selector (one v_perm_b32: the word a where the lane's bit is set,
// else b); written as selects, the compiler turns them into selects of
// array addresses, and the arrays into scratch.
__device__ __forceinline__ uint32_t blend(uint32_t sel, uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(a, b, sel); }

__device__ __forceinline__ void quad_transpose(uint32_t (&h)[4][8], uint32_t lane) {
    const uint32_t m0 = lane & 1u ? 0x07060504u : 0x03020100u, m1 = lane & 2u ? 0x07060504u : 0x03020100u;
    // stage on lane bit 0 (partner lane ^ 1, quad_perm 1,0,3,2) against rows
    // (0, 1) and (2, 3): the lane with bit 0 clear keeps row a and takes its
    // partner's row a into row a + 1; the other keeps row a + 1 and takes its
    // partner's row a + 1 into row a. (Every source lane of a quad_perm is
    // valid, so the DPP moves have no old value to keep.)
#pragma unroll
    for (int w = 0; w < 8; ++w) {
#pragma unroll
        for (int a = 0; a < 4; a += 2) {
            const uint32_t u0 = __builtin_amdgcn_mov_dpp(h[a][w], 0xB1, 0xF, 0xF, true);
            const uint32_t u1 = __builtin_amdgcn_mov_dpp(h[a + 1][w], 0xB1, 0xF, 0xF, true);
            h[a][w] = blend(m0, u1, h[a][w]);
            h[a + 1][w] = blend(m0, h[a + 1][w], u0);
        }
    }
    // the same on lane bit 1 (partner ^ 2, quad_perm 2,3,0,1), rows (0, 2), (1, 3)
#pragma unroll
    for (int w = 0; w < 8; ++w) {
#pragma unroll
        for (int a = 0; a < 2; ++a) {
            const uint32_t u0 = __builtin_amdgcn_mov_dpp(h[a][w], 0x4E, 0xF, 0xF, true);
            const uint32_t u2 = __builtin_amdgcn_mov_dpp(h[a + 2][w], 0x4E, 0xF, 0xF, true);
            h[a][w] = blend(m1, u2, h[a][w]);
            h[a + 2][w] = blend(m1, h[a + 2][w], u0);
        }
    }
}

// The eight pair words of a decoded block, required in registers here:
// ordered before the next volatile statement (the refill of the stage the
// block came from), so its decode is not deferred past that load and the
// stage's old and new registers never overlap (which would take copies of
// registers whose loads are still in flight).
__device__ __forceinline__ void settle(const uint32_t (&h)[8]) {
    asm volatile("" ::"v"(h[0]), "v"(h[1]), "v"(h[2]), "v"(h[3]), "v"(h[4]), "v"(h[5]), "v"(h[6]), "v"(h[7]));
}

// One quad step's products: the transposed rows h against the activation
// rows at xq (the lane's A address in the step's column block: activation
// row lane % 4, chunk 4 (lane / 4); chunk c of a 1024-column block holds
// columns 16c .. 16c + 7, chunk 64 + c columns 16c + 8 .. 16c + 15), rows
// 4g .. 4g + 3 of the activation into d[g] (even and odd MFMAs into
// separate chains). x4 is four activation rows' LDS stride in bytes.
template <int G>
__device__ __forceinline__ void quad_mfma(f32x4 (&d)[G][2], const uint8_t* xq, uint32_t x4, const uint32_t (&h)[4][8]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            // MFMAs s = 4r + 2 half, + 1: columns 64b + 16r + 8 half .. + 7
            const bf16x4_t b0 = __builtin_bit_cast(bf16x4_t, make_uint2(h[r][4 * half], h[r][4 * half + 1]));
            const bf16x4_t b1 = __builtin_bit_cast(bf16x4_t, make_uint2(h[r][4 * half + 2], h[r][4 * half + 3]));
#pragma unroll
            for (int g = 0; g < G; ++g) {
                uint4 a;
                __builtin_memcpy(&a, xq + g * x4 + 1024 * half + 16 * r, 16);
                d[g][0] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(bf16x4_t, make_uint2(a.x, a.y)), b0,
                                                               d[g][0], 0, 0, 0);
                d[g][1] = __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(bf16x4_t, make_uint2(a.z, a.w)), b1,
                                                               d[g][1], 0, 0, 0);
            }
        }
    }
}

// A quad unit's sums: lane 4b + j's chains summed, then over the 16 quads b
// (a fixed butterfly: every lane of a residue class gets the same bits);
// lane j < 4 stores output row 4q + j's sums for activation rows 4g + i into
// red[(slot0 + j S) M + 4g + i] where that row is in the tile. The chains are
// cleared.
template <int M, int G>
__device__ __forceinline__ void quad_unit_end(f32x4 (&d)[G][2], float* red, uint32_t slot0, uint32_t segs,
                                              uint32_t row0, uint32_t nrows, uint32_t lane) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        f32x4 s = d[g][0] + d[g][1];
#pragma unroll
        for (int k = 4; k < 64; k <<= 1)
#pragma unroll
            for (int i = 0; i < 4; ++i) s[i] += __shfl_xor(s[i], k, kWave);
        if (lane < 4 && row0 + lane < nrows) {
#pragma unroll
            for (int i = 0; i < 4; ++i) red[(slot0 + lane * segs) * M + 4 * g + i] = s[i];
        }
        d[g][0] = d[g][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
}

// A group of sip tensors that share the activation (the q/k/v or gate/up
// projections of a layer) runs as one launch: their rows form one row
// space, tensor i's from row0[i]. The host keeps the row tile no taller than
// the group's shortest tensor, so a workgroup's rows span at most two
// tensors; such a workgroup holds both tensors' exponent tables. One tensor
// is the group of one.
struct SipGroup {
    const uint32_t* data[kGroupMax];
    const uint32_t* offsets[kGroupMax];
    const uint32_t* palette[kGroupMax];
    const void* bias[kGroupMax];
    void* out[kGroupMax];
    uint32_t row0[kGroupMax + 1];  // row0[n] = the group's row count
};
static_assert(sizeof(SipGroup) + 8 + sizeof(SipShape) <= 5 * 64, "the sip and gulp arguments span five lines");

// arr[i] for a wave-uniform i < kGroupMax, by selects (no indexed copy of
// the kernel arguments).
template <typename T>
__device__ __forceinline__ T pick(const T (&arr)[kGroupMax], uint32_t i) {
    T v = arr[0];
#pragma unroll
    for (int k = 1; k < kGroupMax; ++k) v = i == (uint32_t)k ? arr[k] : v;
    return v;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct SipStage {
    u32x4 lit;
    u32x2 t0;
    uint32_t term;
    uint32_t start, end;
    uint32_t t;  // 0: the workgroup's first tensor, 1: its second
    u32x4 hi;    // raw twin: the lane's weights 16l + 8 .. 16l + 15 (lit holds 16l .. 16l + 7)
};

// The directory, read-only for the whole launch: through the constant
// address space its wave-uniform reads become scalar loads.
typedef const __attribute__((address_space(4))) uint32_t* const_u32_ptr;

// The kernel arguments of the sip and gulp kernels (SipGroup, x, SipShape:
// 296 bytes) lie in five 64-byte lines of the argument segment. The
// prologue reads them in several batches, each waited on before the next
// (the placement needs the shape, the tensor pointers need the placement),
// and each batch's first read of a line costs a round trip to memory.
// Reading one word of every line here, in one batch with one wait, brings
// them all into the scalar cache at once; the later reads hit there.
__device__ __forceinline__ void touch_kernel_args() {
    const const_u32_ptr ka = (const_u32_ptr)__builtin_amdgcn_kernarg_segment_ptr();
    const uint32_t a0 = ka[0], a1 = ka[16], a2 = ka[32], a3 = ka[48], a4 = ka[64];
    asm volatile("" ::"s"(a0), "s"(a1), "s"(a2), "s"(a3), "s"(a4));
}

// A block's directory pair, read through the scalar cache. (The byte
// offset is 32-bit, so the load takes it in an SGPR with no 64-bit address
// add: the fast kernels run tensors of fewer than 2^30 blocks.)
__device__ __forceinline__ uint2 sip_offsets(const uint32_t* offsets, uint32_t blk) {
    const const_u32_ptr p = (const_u32_ptr)(reinterpret_cast<const char*>(offsets) + blk * 4u);
    return make_uint2(p[0], p[1]);
}


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

// A block's loads, non-temporal (`nt`): a sweep reads each weight once, and
// keeping the stream out of the caches measured 2.7% faster on the Qwen3-8B
// step: the terminal word, the tier-0 pair and the literals, issued as one
// unit of three vector loads. They are written as instructions the compiler
// does not track, so the only waits on them are the explicit SIP_WAIT
// below, placed where a stage is consumed: loads return in issue order, so
// waiting until at most N newer loads are outstanding completes the stage,
// whatever other loads the compiler adds after it.
// The terminal goes through a buffer resource spanning the block alone
// ([start, end) of its directory pair): a lane past the block's last word
// reads 0 and fetches nothing. That keeps the next block's literals from
// being fetched twice (the traffic was 7% above the block bytes that way;
// bitwise the same outputs, the Qwen3-8B step 3.2% faster). The literal
// and tier-0 reads (the block's first 352 words) go through one from the
// block's start with no end, as drinkme's readers take a block cut shorter
// than that: the words after it. A stage past the wave's work comes with a
// zero-length pair (end = start) and both resources empty: nothing of it
// is fetched, and the stage is only waited on.
__device__ __forceinline__ SipStage sip_load(uint2 o, uint32_t t, const SipLanes& ln, const uint32_t* data) {
    SipStage s;
    s.start = o.x;
    s.end = o.y;
    s.t = t;
    const i32x4 rterm = make_rsrc(data + o.x, (o.y - o.x) * 4u);
    i32x4 rfix = rterm;
    rfix.z = o.y != o.x ? 0x7FFFFFFF : 0;
    asm volatile(
        "buffer_load_dword %0, %3, %6, 0 offen nt\n\t"
        "buffer_load_dwordx2 %1, %4, %7, 0 offen nt\n\t"
        "buffer_load_dwordx4 %2, %5, %7, 0 offen nt"
        : "=&v"(s.term), "=&v"(s.t0), "=&v"(s.lit)
        : "v"(ln.term), "v"(ln.t0), "v"(ln.lit), "s"(rterm), "s"(rfix));
    return s;
}

// Completes stage S: at most N vector loads issued after it still in flight.
// The "+v" operands make S's registers this statement's results, so nothing
// reads them before the wait.
#define SIP_WAIT(N, S) asm volatile("s_waitcnt vmcnt(" #N ")" : "+v"(S.lit), "+v"(S.t0), "+v"(S.term))

// The raw twin's block: lane l's 16 bf16 weights, 32 bytes at byte offset
// `off` of the workgroup's first row plus 32 l, as two 128-bit loads (word
// j of the pair = weights 16l + 2j, 16l + 2j + 1: the pair words the decode
// builds). Untracked like the payload loads: completed by RAW_WAIT.
__device__ __forceinline__ SipStage raw_load(i32x4 rsrc, uint32_t off, const SipLanes& ln) {
    SipStage s;
    s.start = s.end = s.t = 0;
    asm volatile(
        "buffer_load_dwordx4 %0, %2, %3, %4 offen nt\n\t"
        "buffer_load_dwordx4 %1, %2, %3, %4 offen offset:16 nt"
        : "=&v"(s.lit), "=&v"(s.hi)
        : "v"(ln.raw), "s"(rsrc), "s"(off));
    return s;
}

#define RAW_WAIT(N, S) asm volatile("s_waitcnt vmcnt(" #N ")" : "+v"(S.lit), "+v"(S.hi))

// What a block in flight is, taken from the cursor when its loads are
// issued (so no second cursor walks behind the loads): its unit's row
// partial, its column block among the resident activations, its tensor
// among the workgroup's two, its column phase, and whether it closes its
// unit.
struct SipRef {
    uint32_t slot, cb, t, p;  // (decode mode: t is the block's index in its tensor, the output's block)
    uint32_t row;             // quad mode: the quad's first row in the tile
    bool last;
};

// Rows 0..M-1 of x, columns [phase K 1024, (phase + 1) K 1024), into LDS
// by direct loads: row m at xs + m xrow; within each 1024-column block,
// 16-byte chunk q < 64 holds x[16q .. 16q + 7] and chunk 64 + q holds
// x[16q + 8 .. 16q + 15], so a lane's two reads of its 16 activations each
// cover 1 KB contiguously over the wave (no bank conflicts). A padding row
// (m >= sh.m) repeats the last real row (its sums are never stored).
//
// The loads are written as instructions the compiler does not track (as the
// payload loads are), so it adds no wait of its own for them: the caller
// waits with an explicit vmcnt before the barrier that publishes xs. Each
// wave loads whole 64-chunk runs (row_chunks is a multiple of 64), so M0,
// the wave's LDS destination, is uniform. M0 is the compiler's register:
// the statement restores it, and waits the one state an M0 write needs
// before an LDS-bound load reads it.
__device__ __forceinline__ void lds_load16(const void* g, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(g), "s"(lds)
        : "memory");
}

// THREADS: the workgroup's threads (a wave-uniform value)
template <int M>
__device__ __forceinline__ void load_x_slice(const SipShape& sh, const uint16_t* __restrict__ x, uint16_t* xs,
                                             uint32_t phase, uint32_t THREADS) {
    const uint32_t lane = lane_id(), wbase = wave_id() * 64u;
    const uint32_t row_chunks = sh.phase_blocks * 128u, xchunks = sh.cols / 8, first = phase * row_chunks;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)xs;
#pragma unroll
    for (uint32_t m = 0; m < (uint32_t)M; ++m) {
        const uint32_t src_row = min(m, sh.m - 1) * xchunks + first;
        for (uint32_t jw = wbase; jw < row_chunks; jw += THREADS) {
            const uint32_t j = jw + lane;
            const uint32_t q = j & 127u, src = src_row + ((j & ~127u) | (q < 64u ? 2u * q : 2u * (q - 64u) + 1u));
            lds_load16(reinterpret_cast<const uint4*>(x) + src, lds0 + 2u * m * sh.xrow + 16u * jw);
        }
    }
}

// Builds the exponent table of a palette: entry g (four 3-bit codes c0..c3)
// holds E(c0) << 7 | E(c1) << 23 | m << 3 and E(c2) << 7 | E(c3) << 23, where
// E(7) = 0 (the pad byte) and m = the four escape flags.
__device__ __forceinline__ void sip_table(uint2* tb, const uint32_t* palette) {
    const uint32_t p0 = ((const_u32_ptr)palette)[0], p1 = ((const_u32_ptr)palette)[1];
    // thread h < 512 writes entries 8h .. 8h + 7: c1 c2 c3 = h's codes, c0 = 0..7
    const uint32_t h = threadIdx.x;
    if (h < 512) {
        const uint32_t c1 = h & 7, c2 = (h >> 3) & 7, c3 = h >> 6;
        const uint32_t y = ((__builtin_amdgcn_perm(p1, p0, c2) & 0xFF) << 7) | ((__builtin_amdgcn_perm(p1, p0, c3) & 0xFF) << 23);
        const uint32_t xb = ((__builtin_amdgcn_perm(p1, p0, c1) & 0xFF) << 23) |
                            ((((c1 == 7) << 1) | ((c2 == 7) << 2) | ((c3 == 7) << 3)) << 3);
#pragma unroll
        for (uint32_t c0 = 0; c0 < 8; c0 += 2) {
            const uint32_t e0 = c0 < 4 ? (p0 >> (8 * c0)) & 0xFF : (p1 >> (8 * (c0 - 4))) & 0xFF;
            const uint32_t e1 = c0 + 1 < 4 ? (p0 >> (8 * (c0 + 1))) & 0xFF : (p1 >> (8 * (c0 - 3))) & 0xFF;
            const uint4 v = make_uint4(xb | (e0 << 7), y, xb | (e1 << 7) | ((c0 + 1 == 7) << 3), y);
            *reinterpret_cast<uint4*>(tb + 8 * h + c0) = v;
        }
    }
}

// TWO: some workgroup of the launch spans two tensors (the instantiation
// without it carries no per-block tensor selects). M: activation rows, 1, 2,
// 4 or 8 (sh.m of them real); each decoded weight pair meets the M rows in
// turn, so the decode is paid once per block whatever M is.
// (M = 8 holds one workgroup per CU: its activation rows alone take 8 * 2 *
// cols bytes of LDS, so it is given the registers of 3 waves per SIMD.)
// PH: the activation columns come in phases (sh.phases > 1), for rows too
// long for LDS; the other instantiations carry no phase code. (With M = 4
// too, it keeps one workgroup per CU, for the registers.)
// MODE: 0 the GEMV; 1, 2 the raw twin (the decode replaced by a load of the
// raw weight) mirroring the sip or the gulp kernel's matrix-core rule; 3
// decode only: each block's bf16 bits stored to the tensor's output
// (row-major [rows, cols]) in place of the products.
constexpr int kModeGemv = 0, kModeTwinSip = 1, kModeTwinGulp = 2, kModeDecode = 3;
constexpr int kModeTwinGulpMx = 4;  // the raw twin of gulp under the matrix policy

template <bool TWO, int M, bool PH, int MODE = kModeGemv>
__global__ __launch_bounds__(kSipThreads, (M == 8 || (M == 4 && (MODE == kModeTwinGulp ? gulp_quad(4) : MODE == kModeTwinGulpMx ? gulp_quad(4, true) : (PH || sip_quad(4))))) ? 3 : 6)
void k_gemv_sip(const SipGroup g, const uint16_t* __restrict__ x, const SipShape sh) {
    constexpr bool RAW = MODE == kModeTwinSip || MODE == kModeTwinGulp || MODE == kModeTwinGulpMx;
    constexpr bool DEC = MODE == kModeDecode;
    // verify rows four output rows at a time on the matrix cores (a raw twin
    // mirroring gulp: gulp's rule)
    constexpr bool QUAD = !DEC && (MODE == kModeTwinGulp    ? gulp_quad(M)
                                   : MODE == kModeTwinGulpMx ? gulp_quad(M, true)
                                                             : sip_quad(M));
    static_assert(!(TWO && MODE), "the raw twin and the decode run one tensor");
    static_assert(!DEC || (M == 1 && !PH), "the decode runs unphased");
    // fixed-size tables in static LDS (their addresses fold into the LDS
    // instructions' offsets); the activation, the row partials and a second
    // tensor's table after them
    __shared__ uint2 tbl[4096];
    __shared__ uint2 sel[16];
    __shared__ uint32_t wg_done;  // blocks the workgroup's waves have started (progress balance)
    __shared__ uint2 sel2[13 * 16];
    extern __shared__ __align__(16) uint8_t lds_dyn[];
    touch_kernel_args();
    uint16_t* xs = reinterpret_cast<uint16_t*>(lds_dyn);
    // (a multiple of 8 bf16, stated so that 16-byte LDS reads of the rows stay whole)
    const uint32_t xrow = sh.xrow & ~7u;
    float* red = reinterpret_cast<float*>(lds_dyn + 2 * M * xrow);
    uint2* tbl2 = reinterpret_cast<uint2*>(lds_dyn + sh.tbl2_lds);

    const uint32_t wv = wave_id(), lane = lane_id();
    // the workgroup's tensors: ia holds its first row; rows [split, nrows)
    // are ib's
    const WgPlace wp0 = wg_place<TWO>(sh, g.row0, blockIdx.x);
    const uint32_t nrows = wp0.nrows, ia = wp0.ia, ib = wp0.ib, row_a = wp0.row_a, row_b = wp0.row_b;
    const uint32_t split = wp0.split, lrow_a = wp0.lrow_a;
    const SipSpan sp = wp0.sp;
    const uint32_t units = (QUAD ? (nrows + 3) / 4 : nrows) * sh.segs;
    const bool two = TWO && split < nrows;
    const uint32_t* data_a = pick(g.data, ia);
    const uint32_t* data_b = pick(g.data, ib);
    const uint32_t* offsets_a = pick(g.offsets, ia);
    const uint32_t* offsets_b = pick(g.offsets, ib);

    // the activation (its first column phase) goes to LDS by direct loads
    // (no registers staged), first in the queue: small and hot in L2; the
    // barrier below waits for it
    if constexpr (!DEC) load_x_slice<M>(sh, x, xs, 0, kSipThreads);

    // the first two blocks' loads go out before the tables are built; a
    // cursor past the wave's work reads the workgroup's first directory
    // entry and, through a zero-length window, no payload
    SipCursor p;
    QuadCursor pq;
    const SipWalk wk = sip_walk<QUAD>(sh, nrows);
    if constexpr (QUAD)
        quad_start(sh, pq, wv, wk);
    else
        sip_start<TWO>(sh, p, wv, wk, sp);
    SipRef nr;  // the last next_offsets() block
    auto next_offsets = [&]() {
        Issue is;
        if constexpr (QUAD) {
            // (the four blocks of a quad step share its column block, phase
            // and unit: row 4q's partial is slot, row 4q + j's slot + j S)
            is = quad_issue<TWO>(sh, pq, sp, nrows);
            nr.t = is.t;
            nr.row = 4 * pq.q;
            nr.slot = nr.row * sh.segs + pq.p * sh.psegs + pq.sp;
            nr.cb = pq.sp * sh.seg_blocks + pq.c;
            nr.p = pq.p;
            nr.last = pq.c + 1 == sh.seg_blocks;
        } else {
            is = sip_issue<TWO>(sh, p, sp);
            nr.t = DEC ? p.blk : is.t;
            nr.slot = p.slot;
            nr.cb = p.cb;
            nr.p = p.p;
            nr.last = p.j + 1 == sh.seg_blocks;
        }
        uint2 o;
        if constexpr (RAW) {  // the block's byte offset from the workgroup's first row
            o = make_uint2((is.blk - sp.a_first) * 2048u, 0u);
        } else {
            o = sip_offsets(TWO && is.t ? offsets_b : offsets_a, is.blk);
            if (!is.live) o.y = o.x;  // (past the work: a zero-length window, nothing fetched)
        }
        if constexpr (QUAD)
            quad_next(sh, pq, wk);
        else
            sip_next<TWO>(sh, p, wk, sp);
        return o;
    };
    // the first blocks' directory entries, all issued before any is waited
    // on (one round trip)
    const uint2 oA = next_offsets();
    SipRef rA = nr;
    const uint2 oB = next_offsets();
    SipRef rB = nr;
    uint2 oC = next_offsets();
    SipRef rC = nr;
    uint2 oD = make_uint2(0u, 0u);
    SipRef rD;
    if constexpr (QUAD) {
        oD = next_offsets();
        rD = nr;
    }
    // the raw twin's window: from the workgroup's first row, 512 words a
    // block (the compressed blocks load through windows of their own)
    const i32x4 rsrc_a = make_rsrc(data_a + (uint64_t)sp.a_first * 512u, 0x7FFFFFFFu);
    const SipLanes ln = sip_lanes(lane);
    auto load = [&](uint2 o, uint32_t t) {
        if constexpr (RAW) return raw_load(rsrc_a, o.x, ln);
        return TWO && t ? sip_load(o, 1u, ln, data_b) : sip_load(o, 0u, ln, data_a);
    };
    // the prologue's stages issue in the loop's order (no interleaving),
    // so the waits the loop needs are the same on entry as in steady state
    SipStage sA = load(oA, rA.t);
    __builtin_amdgcn_sched_barrier(0);
    SipStage sB = load(oB, rB.t);
    __builtin_amdgcn_sched_barrier(0);
    // M >= 4 keeps three blocks in flight through its longer per-block work
    // (measured 2-4% faster on Qwen3-8B and 32B-class layers at M = 4 over
    // two A/B runs; at M = 1 the same pipeline was 1.7% slower on the step
    // and 6% on 4096 x 4096; at M = 2, mixed)
    constexpr bool DEEP = M >= 4;
    SipStage sC, sD;
    if constexpr (DEEP) {
        sC = load(oC, rC.t);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (QUAD) {  // (quad steps keep four blocks in flight: one step's)
        sD = load(oD, rD.t);
        __builtin_amdgcn_sched_barrier(0);
    }

    if constexpr (!RAW) {
    sip_table(tbl, pick(g.palette, ia));
    if (two) sip_table(tbl2, pick(g.palette, ib));
    // selectors of escape mask m (4 weights) at offset o: byte 0 / 2 of word
    // k / 2 picks, for weight k of the group, the window byte of its escape
    // (o + its rank among the group's escapes), or 0x0C (a zero byte) when
    // k did not escape. sel: o = 0 (a window per group); sel2[o][m]: one
    // 8-byte window per lane, o = the lane's escapes in earlier groups.
    for (uint32_t i = threadIdx.x; i < 13 * 16; i += kSipThreads) {
        const uint32_t m = i & 15, o = i >> 4;
        uint32_t b[4];
        for (uint32_t k = 0, r = o; k < 4; ++k) b[k] = (m >> k) & 1 ? (r++ & 7) : 0x0Cu;
        const uint2 e = make_uint2(b[0] | 0x0C00u | (b[1] << 16) | 0x0C000000u,
                                   b[2] | 0x0C00u | (b[3] << 16) | 0x0C000000u);
        sel2[i] = e;
        if (o == 0) sel[m] = e;
    }
    }
    // every wave's direct loads into LDS must land before any wave reads:
    // they precede the two stages' 6 loads (raw: 4) in the wave's queue, so
    // vmcnt(6) completes them while the stages stay in flight
    if (threadIdx.x == 0) wg_done = 0;
    if constexpr (RAW && QUAD)
        asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if constexpr (QUAD)
        asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else if constexpr (RAW && DEEP)
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    else if constexpr (RAW)
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    else if constexpr (DEEP)
        asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    __syncthreads();

    const uint32_t keep = 0x807F807Fu;  // sign + mantissa bits of a bf16 pair, from the literal
    // M = 1 keeps two accumulator chains; M > 1 one per row
    float acc0 = 0.0f, acc1 = 0.0f;
    // verify rows on the matrix cores (a raw twin mirroring gulp: gulp's rule)
    constexpr int MA = QUAD ? 1 : M;  // v_dot2 rows (the quad path accumulates on the matrix cores)
    float acc[MA];
#pragma unroll
    for (int m = 0; m < MA; ++m) acc[m] = 0.0f;
    // quad mode: activation rows 4g .. 4g + 3 meet the four output rows in
    // chains dq[g] (even and odd MFMAs)
    constexpr int G = QUAD ? M / 4 : 1;
    f32x4 dq[G][2];
#pragma unroll
    for (int g2 = 0; g2 < G; ++g2) dq[g2][0] = dq[g2][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // one block of the wave's work, from its loaded stage
    // column phases: every wave walks all of them in order (so the barriers
    // match); a phase's activations replace the last one's once every wave
    // is past it
    uint32_t cur_phase = 0;
    auto phase_advance = [&]() {
        __syncthreads();
        ++cur_phase;
        load_x_slice<M>(sh, x, xs, cur_phase, kSipThreads);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    // (quad mode: the block's pair words go to hout, and the quad step does
    // the products)
    auto process = [&](const SipStage& s0, const SipRef& c, uint32_t* hout) {
        if (PH && !QUAD)
            while (cur_phase < c.p) phase_advance();
        const uint16_t* xb;
        uint4 xa, xc;
        uint32_t wp[8];
        if constexpr (RAW) {
            // the twin: the lane's raw pair words in place of the decode
            xb = xs + c.cb * 1024 + 8 * lane;
            if (M == 1) {
                __builtin_memcpy(&xa, xb, 16);
                __builtin_memcpy(&xc, xb + 512, 16);
            }
            wp[0] = s0.lit.x;
            wp[1] = s0.lit.y;
            wp[2] = s0.lit.z;
            wp[3] = s0.lit.w;
            wp[4] = s0.hi.x;
            wp[5] = s0.hi.y;
            wp[6] = s0.hi.z;
            wp[7] = s0.hi.w;
        } else {
        const uint2* tb = TWO && s0.t ? tbl2 : tbl;
        const uint64_t v = ((uint64_t)s0.t0.y << 32 | s0.t0.x) >> ((lane & 1) * 16);
        const uint32_t lo = (uint32_t)v, hi = (uint32_t)(v >> 32);
        uint2 E0 = tb[lo & 0xFFF];
        uint2 E1 = tb[(lo >> 12) & 0xFFF];
        uint2 E2 = tb[__builtin_amdgcn_alignbit(hi, lo, 24) & 0xFFF];
        uint2 E3 = tb[(hi >> 4) & 0xFFF];
        xb = xs + c.cb * 1024 + 8 * lane;
        if (M == 1) {
            __builtin_memcpy(&xa, xb, 16);
            __builtin_memcpy(&xc, xb + 512, 16);
        }

        // escapes: group g's flags are bits 3..6 of E_g.x (a_g = m_g << 3);
        // a lane's escapes are terminal bytes q0 .. q0 + cnt - 1
        const uint32_t a0 = E0.x & 0x78u, a1 = E1.x & 0x78u, a2 = E2.x & 0x78u, a3 = E3.x & 0x78u;
        const uint32_t q1_ = __builtin_popcount(a0), q2_ = q1_ + __builtin_popcount(a1);
        const uint32_t q3_ = q2_ + __builtin_popcount(a2), cnt = q3_ + __builtin_popcount(a3);
        // the groups' selectors depend only on the lane's own counts: read
        // them before the scan, so their LDS round trip overlaps the
        // cross-lane reads' (a lane with up to 16 escapes indexes rows up
        // to 12 of sel2)
        const uint2 sl0 = sel2[a0 >> 3], sl1 = sel2[(q1_ << 4) | (a1 >> 3)];
        const uint2 sl2 = sel2[(q2_ << 4) | (a2 >> 3)], sl3 = sel2[(q3_ << 4) | (a3 >> 3)];
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t inc = wave_scan_incl(cnt), q0 = inc - cnt;
        // the terminal is read only when the directory gives the block words
        // past its fixed streams (radix_kernel_gpu.py:96-98); without it the
        // escaped exponents stay 0
        const bool has_term = s0.end > s0.start + kSipFixed;
        const uint32_t tw = has_term ? s0.term : 0u;  // lane j: terminal word j
        // every lane takes the windowed patch, exact where the lane has at
        // most 8 escapes, all in terminal words 0..62 (the common case); the
        // window's three words come from the lanes holding them
        const int k0 = (int)(q0 & ~3u);
        const uint32_t w0 = __builtin_amdgcn_ds_bpermute(k0, tw);
        const uint32_t w1 = __builtin_amdgcn_ds_bpermute(k0 + 4, tw);
        const uint32_t w2 = __builtin_amdgcn_ds_bpermute(k0 + 8, tw);
        const uint32_t wlo = __builtin_amdgcn_alignbit(w1, w0, q0 << 3);
        const uint32_t whi = __builtin_amdgcn_alignbit(w2, w1, q0 << 3);
#define DMX_PATCH2(E, s)                                \
    {                                                   \
        E.x |= __builtin_amdgcn_perm(whi, wlo, s.x) << 7; \
        E.y |= __builtin_amdgcn_perm(whi, wlo, s.y) << 7; \
    }
        DMX_PATCH2(E0, sl0)
        DMX_PATCH2(E1, sl1)
        DMX_PATCH2(E2, sl2)
        DMX_PATCH2(E3, sl3)
#undef DMX_PATCH2
        // rare: a lane with more than 8 escapes, or more than 243 before it,
        // redoes its exponents with each group's four bytes read from the
        // terminal stream in memory (at most word 352 + 257 of the block:
        // inside the reach pad). Without a terminal the window was zero and
        // every lane is already exact. So does every lane of a block whose
        // terminal is shorter than its escapes (a malformed block the gate
        // passes): its loaded words stop at the block's end, and the bytes
        // past it are the following words, as a reader without an end bound
        // takes them.
        const bool short_term = has_term && __builtin_amdgcn_readlane(inc, 63) > 4u * (s0.end - s0.start - kSipFixed);
        const bool wide = cnt > 8 || q0 > 243 || short_term;
        if (__builtin_expect(__builtin_amdgcn_ballot_w64(wide) != 0, 0) && has_term && wide) {
            E0 = tb[lo & 0xFFF];
            E1 = tb[(lo >> 12) & 0xFFF];
            E2 = tb[__builtin_amdgcn_alignbit(hi, lo, 24) & 0xFFF];
            E3 = tb[(hi >> 4) & 0xFFF];
            const uint32_t* tp = (TWO && s0.t ? data_b : data_a) + s0.start + kSipFixed;
#define DMX_PATCH(E, a, qoff)                                                   \
    {                                                                           \
        const uint32_t q = q0 + (qoff);                                         \
        const uint2 s = sel[(a) >> 3];                                          \
        const uint32_t w = __builtin_amdgcn_alignbit(tp[(q >> 2) + 1], tp[q >> 2], q << 3); \
        E.x |= __builtin_amdgcn_perm(0u, w, s.x) << 7;                          \
        E.y |= __builtin_amdgcn_perm(0u, w, s.y) << 7;                          \
    }
            DMX_PATCH(E0, a0, 0)
            DMX_PATCH(E1, a1, q1_)
            DMX_PATCH(E2, a2, q2_)
            DMX_PATCH(E3, a3, q3_)
#undef DMX_PATCH
        }
        const uint32_t L0 = s0.lit.x, L1 = s0.lit.y, L2 = s0.lit.z, L3 = s0.lit.w;
        wp[0] = (__builtin_amdgcn_perm(L0, L0, 0x01010000) & keep) | (E0.x & ~keep);
        wp[1] = (__builtin_amdgcn_perm(L0, L0, 0x03030202) & keep) | (E0.y & ~keep);
        wp[2] = (__builtin_amdgcn_perm(L1, L1, 0x01010000) & keep) | (E1.x & ~keep);
        wp[3] = (__builtin_amdgcn_perm(L1, L1, 0x03030202) & keep) | (E1.y & ~keep);
        wp[4] = (__builtin_amdgcn_perm(L2, L2, 0x01010000) & keep) | (E2.x & ~keep);
        wp[5] = (__builtin_amdgcn_perm(L2, L2, 0x03030202) & keep) | (E2.y & ~keep);
        wp[6] = (__builtin_amdgcn_perm(L3, L3, 0x01010000) & keep) | (E3.x & ~keep);
        wp[7] = (__builtin_amdgcn_perm(L3, L3, 0x03030202) & keep) | (E3.y & ~keep);
        }
        if constexpr (DEC) {
            // the lane's 16 weights: 32 bytes at weight 1024 blk + 16 lane
            uint4* d = reinterpret_cast<uint4*>(pick(g.out, ia)) + (uint64_t)c.t * 128u + 2u * lane;
            d[0] = make_uint4(wp[0], wp[1], wp[2], wp[3]);
            d[1] = make_uint4(wp[4], wp[5], wp[6], wp[7]);
            return;
        }
        if constexpr (QUAD) {
            if constexpr (RAW) {
                // the raw twin's words are the stage's own registers, refilled
                // next: copied out now, after the stage's wait
#pragma unroll
                for (int i = 0; i < 8; ++i) asm volatile("v_mov_b32 %0, %1" : "=v"(hout[i]) : "v"(wp[i]));
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) hout[i] = wp[i];
            }
            return;
        }
        if (M == 1) {
            acc0 = dot2(wp[0], xa.x, acc0);
            acc1 = dot2(wp[1], xa.y, acc1);
            acc0 = dot2(wp[2], xa.z, acc0);
            acc1 = dot2(wp[3], xa.w, acc1);
            acc0 = dot2(wp[4], xc.x, acc0);
            acc1 = dot2(wp[5], xc.y, acc1);
            acc0 = dot2(wp[6], xc.z, acc0);
            acc1 = dot2(wp[7], xc.w, acc1);
        } else {
#pragma unroll
            for (int m = 0; m < MA; ++m) {
                uint4 ya, yc;
                __builtin_memcpy(&ya, xb + m * xrow, 16);
                __builtin_memcpy(&yc, xb + m * xrow + 512, 16);
                float a = acc[m];
                a = dot2(wp[0], ya.x, a);
                a = dot2(wp[1], ya.y, a);
                a = dot2(wp[2], ya.z, a);
                a = dot2(wp[3], ya.w, a);
                a = dot2(wp[4], yc.x, a);
                a = dot2(wp[5], yc.y, a);
                a = dot2(wp[6], yc.z, a);
                acc[m] = dot2(wp[7], yc.w, a);
            }
        }

        if (c.last) {
            if (M == 1) {
                const float s = wave_sum_dpp(acc0 + acc1);
                if (lane == 0) red[c.slot] = s;
                acc0 = acc1 = 0.0f;
            } else {
#pragma unroll
                for (int m = 0; m < MA; ++m) {
                    const float s = wave_sum_dpp(acc[m]);
                    if (lane == 0) red[c.slot * M + m] = s;
                    acc[m] = 0.0f;
                }
            }
        }
    };
    // three stages rotate roles (no register copies); each step issues the
    // stage two blocks ahead, then completes the oldest (six loads newer);
    // whole rounds of three blocks, then the remainder
    const uint32_t my_units = wv < units ? (units - wv + kSipWaves - 1) / kSipWaves : 0;
    const uint32_t items = my_units * sh.seg_blocks * (QUAD ? 4 : 1);
    const uint32_t wg_items = units * sh.seg_blocks;
    const bool balance = !DEC && M <= 2 && wg_items >= kBalanceMinBlocks * kSipWaves;
    if constexpr (QUAD) {
        // a quad step: the four rows' blocks of one column block, stages A,
        // B, C and D, each completed (nine loads newer: the other three
        // stages; raw: six), decoded, and refilled at once with the block
        // four ahead, the stage keeping its registers (no copies of a load
        // in flight); then the four rows meet the activation rows on the
        // matrix cores. A unit is whole steps: items is a multiple of four.
        uint32_t hq[4][8];
        const uint8_t* xq = reinterpret_cast<const uint8_t*>(xs) + (lane & 3u) * 2u * xrow + 64u * (lane >> 2);
        for (uint32_t k = 0; k < items; k += 4) {
            const SipRef step = rA;  // the step's column block, phase and unit (shared by its four blocks)
            if constexpr (RAW) RAW_WAIT(6, sA); else SIP_WAIT(9, sA);
            process(sA, rA, hq[0]);
            settle(hq[0]);
            uint2 oN = next_offsets();
            rA = nr;
            sA = load(oN, rA.t);
            if constexpr (RAW) RAW_WAIT(6, sB); else SIP_WAIT(9, sB);
            process(sB, rB, hq[1]);
            settle(hq[1]);
            oN = next_offsets();
            rB = nr;
            sB = load(oN, rB.t);
            if constexpr (RAW) RAW_WAIT(6, sC); else SIP_WAIT(9, sC);
            process(sC, rC, hq[2]);
            settle(hq[2]);
            oN = next_offsets();
            rC = nr;
            sC = load(oN, rC.t);
            if constexpr (RAW) RAW_WAIT(6, sD); else SIP_WAIT(9, sD);
            process(sD, rD, hq[3]);
            settle(hq[3]);
            oN = next_offsets();
            rD = nr;
            sD = load(oN, rD.t);
            if (PH)
                while (cur_phase < step.p) phase_advance();
            quad_transpose(hq, lane);
            quad_mfma<G>(dq, xq + step.cb * 2048u, 8u * xrow, hq);
            if (step.last) quad_unit_end<M, G>(dq, red, step.slot, sh.segs, step.row, nrows, lane);
        }
        // in flight now: the four stages, past the wave's work; they land
        // before the end
        if constexpr (RAW) RAW_WAIT(0, sD); else SIP_WAIT(0, sD);
    } else {
    uint32_t k = 0;
    for (; k + 3 <= items; k += 3) {
        if (balance) {
            // Progress balance: the SIMD's arbiter favours its oldest
            // waves, and one workgroup's waves otherwise end up to 6 us
            // apart on a 26 us launch, the CU's loads thinning out as they
            // finish. A wave more than kBalanceMargin blocks (of the
            // workgroup's) behind the workgroup's average progress takes
            // the SIMD first. Scheduling only: the results are unchanged.
            // (Off for launches of under kBalanceMinBlocks blocks a wave,
            // where the atomic's round trip before the loads costs more,
            // and at M = 4 and 8: no gain measured, and its registers
            // would spill there.)
            uint32_t tot = 0;
            if (lane == 0) tot = __hip_atomic_fetch_add(&wg_done, 3u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            tot = __builtin_amdgcn_readfirstlane(tot);
            if (k * wg_items + kBalanceMargin * items < tot * items)
                __builtin_amdgcn_s_setprio(2);
            else
                __builtin_amdgcn_s_setprio(0);
        }
        if constexpr (DEEP) {
            // three in flight: complete the oldest, then issue the block
            // three ahead in its place
            if constexpr (RAW) RAW_WAIT(4, sA); else SIP_WAIT(6, sA);
            process(sA, rA, nullptr);
            uint2 oN = next_offsets();
            rA = nr;
            sA = load(oN, rA.t);
            if constexpr (RAW) RAW_WAIT(4, sB); else SIP_WAIT(6, sB);
            process(sB, rB, nullptr);
            oN = next_offsets();
            rB = nr;
            sB = load(oN, rB.t);
            if constexpr (RAW) RAW_WAIT(4, sC); else SIP_WAIT(6, sC);
            process(sC, rC, nullptr);
            oN = next_offsets();
            rC = nr;
            sC = load(oN, rC.t);
        } else {
        sC = load(oC, rC.t);
        uint2 oN = next_offsets();
        SipRef rN = nr;
        if constexpr (RAW) RAW_WAIT(4, sA); else SIP_WAIT(6, sA);
        process(sA, rA, nullptr);
        sA = load(oN, rN.t);
        rA = rN;
        oN = next_offsets();
        rN = nr;
        if constexpr (RAW) RAW_WAIT(4, sB); else SIP_WAIT(6, sB);
        process(sB, rB, nullptr);
        sB = load(oN, rN.t);
        rB = rN;
        oN = next_offsets();
        rN = nr;
        if constexpr (RAW) RAW_WAIT(4, sC); else SIP_WAIT(6, sC);
        process(sC, rC, nullptr);
        oC = oN;
        rC = rN;
        }
    }
    if constexpr (DEEP) {
        // in flight now: sA (older), sB, then sC (never a block of the wave's)
        if constexpr (RAW) RAW_WAIT(4, sA); else SIP_WAIT(6, sA);
        if (k < items) process(sA, rA, nullptr);
        if constexpr (RAW) RAW_WAIT(2, sB); else SIP_WAIT(3, sB);
        if (k + 1 < items) process(sB, rB, nullptr);
        if constexpr (RAW) RAW_WAIT(0, sC); else SIP_WAIT(0, sC);
    } else {
    // in flight now: sA (older), then sB
    if constexpr (RAW) RAW_WAIT(2, sA); else SIP_WAIT(3, sA);
    if (k < items) process(sA, rA, nullptr);
    if constexpr (RAW) RAW_WAIT(0, sB); else SIP_WAIT(0, sB);
    if (k + 1 < items) process(sB, rB, nullptr);
    }
    }
    if constexpr (DEC) return;  // every load has landed (the waits above)
    if (PH)
        while (cur_phase + 1 < sh.phases) phase_advance();
    __syncthreads();
    // each row's segment partials in order, the bias, one rounding; out is
    // [m, rows of its tensor]
    const void* bias_a = pick(g.bias, ia);
    const void* bias_b = pick(g.bias, ib);
    void* out_a = pick(g.out, ia);
    void* out_b = pick(g.out, ib);
    uint32_t rows_b = g.row0[1] - g.row0[0];
#pragma unroll
    for (int k = 1; k < kGroupMax; ++k) rows_b = ib == (uint32_t)k ? g.row0[k + 1] - g.row0[k] : rows_b;
    const uint32_t rows_a = row_b - row_a;
    for (uint32_t i = threadIdx.x; i < nrows * sh.m; i += kSipThreads) {
        const uint32_t m = i / nrows, t = i - m * nrows;
        float sum = 0.0f;
        for (uint32_t k = 0; k < sh.segs; ++k) sum += red[(t * sh.segs + k) * M + m];
        const bool in_b = t >= split;
        const uint32_t row = in_b ? t - split : lrow_a + t;
        const void* bias = in_b ? bias_b : bias_a;
        if (bias) sum += load_elem(bias, sh.bias_dtype, row);
        store_elem(in_b ? out_b : out_a, sh.out_dtype, (uint64_t)m * (in_b ? rows_b : rows_a) + row, sum);
    }
}

// ------------------------------------------------- gulp, M rows, whole blocks --
//
// gulp (2, 2, 4, 8): per 1024-weight block the literal plane (256 words),
// tier 0 (64 words of 2-bit codes: palette entries 0..2, code 3 escapes),
// tier 1 (2-bit codes of the tier-0 escapes: entries 3..5), tier 2 (4-bit
// codes of the tier-1 escapes: entries 6..20) and the terminal (the raw
// exponents of the tier-2 escapes). The streams after tier 0 are short
// (about 24 words a block on normal weights, 28 on Student-t ones), so one
// load of a word a lane brings all three in; their starts follow from the
// block's own counts as the schedule defines them (tier 1 holds the n1
// tier-0 escapes in ceil(n1 / 16) words, tier 2 the n2 tier-1 escapes in
// ceil(n2 / 8)), so the kernel does not read the per-block schedule.
//
// The work split, load pipeline and products are the sip kernel's. Lane l
// owns weights 16l .. 16l + 15; per group of four weights:
//   tier 0  a 256-entry LDS table indexed by the four codes gives the
//           exponents of the resolved weights, the group's tier-1 bit count
//           2 popcount(m0) (m0: its escape mask) and m0's run in the tier-1
//           table;
//   tier 1  the lane's tier-1 codes are a 32-bit window of the tier-1
//           stream at bit 2 q0 (q0: the wave's exclusive prefix of tier-0
//           escape counts), pulled from the lanes holding it (lane j holds
//           tail word j, tier 1 starting at word 0); the group's entry in m0's run of the 625-entry
//           tier-1 table, at its 2 popcount(m0) code bits, gives the tier-1
//           exponents at the escaped positions and the tier-1 escape mask
//           m1;
//   tier 2  lane j resolves tier-1 escapes 2j and 2j + 1 of the block from
//           tier-2 word j / 4 (tail word w1 + j / 4, pulled like tier 1's;
//           and the terminal after tier 2, for code 15) and
//           writes their exponent bytes to the wave's LDS array; each lane
//           reads the 8-byte window of that array at its first rank q1 and
//           places the bytes with the selector table, as sip places its
//           terminal bytes.
// A block with more than 128 tier-1 escapes, or a lane with more than 8,
// or a tail longer than 64 words, or streams past its end, takes an exact
// lane-serial path that reads the streams from memory.


struct GulpStage {
    u32x4 lit;
    uint32_t t0, tail;
    uint32_t len;  // the block's length in words
};


// A lane's buffer offset `off`, or, when it lies past byte `last`, that
// offset with bit 31 set: past the 0x7FFFFFFF records of the workgroup's
// buffer resource, so the lane reads 0 and fetches nothing (offsets here
// stay far below 2^31, so the sign of last - off is the comparison).
__device__ __forceinline__ uint32_t oob_past(uint32_t off, uint32_t last) {
    return off | ((last - off) & 0x80000000u);
}

// The block's three loads through the workgroup's buffer resource (based
// at its first block), untracked by the compiler as in sip_load; completed
// by GULP_WAIT: the literal plane, the tier-0 words and the tail, words
// 320 + lane, which hold tier 1, tier 2 and the terminal back to back
// (their lengths follow from the block's own escape counts; blocks whose
// tail is longer than 64 words take the exact path). Reads reach at most
// word 383 of the block, inside block_word_bounds(1024)[1] = 768. The tail's
// lanes past the block's last word read 0 and fetch nothing (else they load
// the next block's first words, which that block fetches again).
__device__ __forceinline__ GulpStage gulp_load(i32x4 rsrc, uint32_t base, uint2 o, const GulpLanes& ln) {
    GulpStage s;
    s.len = o.y - o.x;
    const uint32_t soff = (o.x - base) * 4u;
    // (the masked offset rides in its load's destination)
    s.tail = oob_past(ln.w, 4u * (o.y - o.x) - 1u - 4u * kGulpFixed);  // (read at offset:1280, word 320)
    asm volatile(
        "buffer_load_dword %0, %0, %3, %4 offen offset:1280 nt\n\t"
        "buffer_load_dword %1, %5, %3, %4 offen offset:1024 nt\n\t"
        "buffer_load_dwordx4 %2, %6, %3, %4 offen nt"
        : "+&v"(s.tail), "=&v"(s.t0), "=&v"(s.lit)
        : "s"(rsrc), "s"(soff), "v"(ln.w), "v"(ln.lit));
    return s;
}

#define GULP_WAIT(N, S) asm volatile("s_waitcnt vmcnt(" #N ")" : "+v"(S.lit), "+v"(S.t0), "+v"(S.tail))

// Field i of width w of the little-endian stream at p, through the vector
// memory path (the lane-serial fallback).
__device__ __forceinline__ uint32_t gulp_field(const uint32_t* p, uint32_t i, uint32_t w) {
    const uint32_t bit = i * w;
    const uint64_t pair = (uint64_t)p[(bit >> 5) + 1] << 32 | p[bit >> 5];
    return (uint32_t)(pair >> (bit & 31u)) & ((1u << w) - 1u);
}

// Builds the gulp tables of a palette (6 words: tier 0, tier 1, tier 2 x 4,
// each entry list padded with a zero byte that the escape code reads; the
// entries are plan.h's gulp_t0_entry and gulp_t1_value, which the host
// model of the walk checks against a direct decode of every code):
//   t0tab[c0 | c1 << 2 | c2 << 4 | c3 << 6]: E(c0) << 7 | E(c1) << 23,
//       E(c2) << 7 | E(c3) << 23, 2 popcount(m0) (the group's tier-1 bits)
//       and 8 t1_base(m0) (the byte offset of m0's run of the tier-1
//       table), each in a word of its own so that neither needs
//       extracting;
//   t1tab[t1_base(m0) + codes]: for a group whose tier-0 escapes are m0,
//       its popcount(m0) tier-1 codes (2 bits each, in order) placed at the
//       escaped positions: E << 7 | E << 23 pairs as tier 0's, with m1 (the
//       positions whose tier-1 code escapes) << 3 | popcount(m1) << 15.
//       m0 has 4^popcount(m0) code patterns, so the runs hold
//       (1 + 4)^4 = 625 entries (a table indexed by m0 and four whole
//       codes would hold 4096, mostly repeats).
//   pal2[c]: tier 2's bytes.
__device__ __forceinline__ void gulp_tables(uint4* t0tab, uint2* t1tab, uint8_t* pal2, const uint32_t* palette,
                                            uint32_t THREADS) {
    const const_u32_ptr pw = (const_u32_ptr)palette;
    const uint32_t p0 = pw[0], p1 = pw[1];
    // (every plan's workgroup has at least 512 threads: one entry each)
    if (threadIdx.x < 256) {
        const uint32_t i = threadIdx.x;
        uint32_t f[4];
        gulp_t0_entry(p0, i, f);
        t0tab[i] = make_uint4(f[0], f[1], f[2], f[3]);
    }
    for (uint32_t i = threadIdx.x; i < kGulpT1Entries; i += THREADS) {
        uint32_t v[2];
        gulp_t1_value(p1, i, v);
        t1tab[i] = make_uint2(v[0], v[1]);
    }
    // (uniform scalar reads: a vector load here would need a vmcnt(0) wait,
    // which would also wait out the payload loads already in flight)
    const uint32_t p2 = pw[2], p3 = pw[3], p4 = pw[4], p5 = pw[5], t = threadIdx.x;
    if (t < 4) reinterpret_cast<uint32_t*>(pal2)[t] = t == 0 ? p2 : t == 1 ? p3 : t == 2 ? p4 : p5;
}

// DEC: decode only, each block's bf16 bits stored to the tensor's output
// (row-major [rows, cols]) in place of the products.
// WV: waves per workgroup, the plan's (12, or 8 at three workgroups per CU).
// MX: the matrix policy (M = 4 in quad units, as M = 8).
template <int M, bool PH, bool DEC = false, int WV = kSipWaves, bool MX = false>
__global__ __launch_bounds__(WV * 64, (M == 8 || (M == 4 && gulp_quad(4, MX))) ? 3 : 6)
void k_gemv_gulp(const SipGroup g, const uint16_t* __restrict__ x, const SipShape sh) {
    static_assert(!DEC || (M == 1 && !PH), "the decode runs unphased");
    static_assert(WV == kSipWaves || (!PH && !DEC && !gulp_quad(M, MX)), "8-wave workgroups run unphased v_dot2 rows");
    constexpr uint32_t W = WV, TH = 64u * WV;
    // verify rows four output rows at a time on the matrix cores
    constexpr bool QUAD = !DEC && gulp_quad(M, MX);
    __shared__ uint4 t0tab[256];
    __shared__ uint2 t1tab[kGulpT1Entries];
    __shared__ uint2 sel2[13 * 16];
    __shared__ uint32_t pal2w[4];
    __shared__ uint32_t x2_all[kSipWaves * kGulpX2Words];
    extern __shared__ __align__(16) uint8_t lds_dyn[];
    touch_kernel_args();
    uint16_t* xs = reinterpret_cast<uint16_t*>(lds_dyn);
    // (a multiple of 8 bf16, stated so that 16-byte LDS reads of the rows stay whole)
    const uint32_t xrow = sh.xrow & ~7u;
    float* red = reinterpret_cast<float*>(lds_dyn + 2 * M * xrow);
    const uint8_t* pal2 = reinterpret_cast<const uint8_t*>(pal2w);

    const uint32_t wv = wave_id(), lane = lane_id();
    // the workgroup's tensor (tiles never span two in this kernel)
    const WgPlace wp0 = wg_place<false>(sh, g.row0, blockIdx.x);
    const uint32_t nrows = wp0.nrows, ia = wp0.ia, row_a = wp0.row_a, row_n = wp0.row_b, lrow = wp0.lrow_a;
    const SipSpan sp = wp0.sp;
    const uint32_t units = (QUAD ? (nrows + 3) / 4 : nrows) * sh.segs;
    const uint32_t* data = pick(g.data, ia);
    const uint32_t* offsets = pick(g.offsets, ia);
    uint32_t* x2 = x2_all + wv * kGulpX2Words;

    // the activation rows (first column phase), as in the sip kernel
    if constexpr (!DEC) load_x_slice<M>(sh, x, xs, 0, TH);

    // p issues the loads, c follows it over the blocks processed (quad mode:
    // pq and cq)
    SipCursor p, c;
    QuadCursor pq, cq;
    const SipWalk wk = sip_walk<QUAD>(sh, nrows);
    if constexpr (QUAD) {
        quad_start(sh, pq, wv, wk);
        cq = pq;
    } else {
        sip_start<false>(sh, p, wv, wk, sp);
        c = p;
    }
    auto next_offsets = [&]() {
        const uint32_t blk = QUAD ? quad_issue<false>(sh, pq, sp, nrows).blk : sip_issue<false>(sh, p, sp).blk;
        const uint2 o = sip_offsets(offsets, blk);
        if constexpr (QUAD)
            quad_next(sh, pq, wk);
        else
            sip_next<false>(sh, p, wk, sp);
        return o;
    };
    // the first blocks' directory entries, then the payload window's base:
    // all issued before any is waited on
    const uint2 oA = next_offsets();
    const uint2 oB = next_offsets();
    uint2 oC = next_offsets();
    uint2 oD0 = make_uint2(0u, 0u);
    if constexpr (QUAD) oD0 = next_offsets();
    const uint32_t base = ((const_u32_ptr)offsets)[sp.a_first];
    const i32x4 rsrc = make_rsrc(data + base, 0x7FFFFFFFu);
    const GulpLanes ln = gulp_lanes(lane);
    GulpStage sA = gulp_load(rsrc, base, oA, ln);
    __builtin_amdgcn_sched_barrier(0);
    GulpStage sB = gulp_load(rsrc, base, oB, ln);
    __builtin_amdgcn_sched_barrier(0);
    GulpStage sC, sD;
    if constexpr (QUAD) {  // (quad steps keep four blocks in flight: one step's)
        sC = gulp_load(rsrc, base, oC, ln);
        __builtin_amdgcn_sched_barrier(0);
        sD = gulp_load(rsrc, base, oD0, ln);
        __builtin_amdgcn_sched_barrier(0);
    }

    gulp_tables(t0tab, t1tab, reinterpret_cast<uint8_t*>(pal2w), pick(g.palette, ia), TH);
    if (threadIdx.x < 13 * 16) {  // (at least 512 threads)
        const uint32_t i = threadIdx.x, m = i & 15, o = i >> 4;
        uint32_t b[4];
        for (uint32_t k = 0, r = o; k < 4; ++k) b[k] = (m >> k) & 1 ? (r++ & 7) : 0x0Cu;
        sel2[i] = make_uint2(b[0] | 0x0C00u | (b[1] << 16) | 0x0C000000u, b[2] | 0x0C00u | (b[3] << 16) | 0x0C000000u);
    }
    // the activation's direct loads precede the stages' loads (two stages:
    // 6; quad mode four: 12)
    if constexpr (QUAD)
        asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else
        asm volatile("s_waitcnt vmcnt(6)" ::: "memory");
    __syncthreads();

    const uint32_t keep = 0x807F807Fu;
    const uint32_t* palg = pick(g.palette, ia);
    float acc0 = 0.0f, acc1 = 0.0f;
    constexpr int MA = QUAD ? 1 : M;  // v_dot2 rows (the quad path accumulates on the matrix cores)
    float acc[MA];
#pragma unroll
    for (int m = 0; m < MA; ++m) acc[m] = 0.0f;
    constexpr int G = QUAD ? M / 4 : 1;  // quad mode: activation rows 4g .. 4g + 3 in chains dq[g]
    f32x4 dq[G][2];
#pragma unroll
    for (int g2 = 0; g2 < G; ++g2) dq[g2][0] = dq[g2][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // column phases: every wave walks all of them in order (so the barriers
    // match); a phase's activations replace the last one's once every wave
    // is past it
    uint32_t cur_phase = 0;
    auto phase_advance = [&]() {
        __syncthreads();
        ++cur_phase;
        load_x_slice<M>(sh, x, xs, cur_phase, TH);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    // (quad mode: the block's pair words go to hout, and the quad step does
    // the products)
    // the first word of the block being processed, from the directory at
    // the block the cursor follows (only the rare paths need it, so no
    // stage keeps it in a register)
    auto block_start = [&]() {
        // (row mode: c.blk rebuilt from the unit and column, which stay live)
        const uint32_t blk = QUAD ? quad_issue<false>(sh, cq, sp, nrows).blk : row_block(sh, c, sp);
        return ((const_u32_ptr)offsets)[blk];
    };
    auto process = [&](const GulpStage& s0, uint32_t* hout) {
        if (PH && !QUAD)
            while (cur_phase < c.p) phase_advance();
        const uint32_t len = s0.len;
        // tier 0
        const uint32_t T0 = s0.t0;
        const uint4 F0 = t0tab[T0 & 0xFF], F1 = t0tab[(T0 >> 8) & 0xFF], F2 = t0tab[(T0 >> 16) & 0xFF],
                    F3 = t0tab[T0 >> 24];
        uint2 E0 = make_uint2(F0.x, F0.y), E1 = make_uint2(F1.x, F1.y), E2 = make_uint2(F2.x, F2.y),
              E3 = make_uint2(F3.x, F3.y);
        // (M = 1 reads its activations late, beside the last lookups: the
        // registers stay free through the tier passes)
        const uint16_t* xb = xs + c.cb * 1024 + 8 * lane;
        uint4 xa, xc;
        // twice the tier-0 escapes of each group, and their prefix in the lane
        const uint32_t o1 = F0.z, o2 = o1 + F1.z, o3 = o2 + F2.z, cnt1 = (o3 + F3.z) >> 1;
        const uint32_t q0 = wave_scan_incl_dpp(cnt1) - cnt1;
        // the tail (lane j holds its word j): tier 1 from word 0, w1 words
        // for the block's n1 tier-0 escapes; tier 2 from word w1
        const uint32_t w1 = (__builtin_amdgcn_readlane(q0 + cnt1, 63) + 15u) >> 4;
        // tier 1: the lane's codes, 2 bits each from bit 2 q0 of the stream
        const int k1 = (int)((q0 >> 2) & ~3u);
        const uint32_t v0 = __builtin_amdgcn_ds_bpermute(k1, s0.tail);
        const uint32_t v1 = __builtin_amdgcn_ds_bpermute(k1 + 4, s0.tail);
        // lane j's two tier-2 codes (tier-1 escapes 2j, 2j + 1, in tier-2
        // word j / 4) and their palette bytes: read beside tier 1's window
        const uint32_t t2w = __builtin_amdgcn_ds_bpermute((int)(ln.t2 + 4u * w1), s0.tail);
        const uint32_t sh2 = (lane & 3u) << 3;
        const uint32_t ca = (t2w >> sh2) & 15u, cb = (t2w >> (sh2 + 4)) & 15u;
        const uint32_t pa = pal2[ca], pb = pal2[cb];
        const uint32_t W1 = __builtin_amdgcn_alignbit(v1, v0, (q0 & 15u) << 1);
        // (the group's 2 popcount(m0) code bits from bit off, at byte
        // offset 8 t1_base(m0) + 8 codes)
#define DMX_T1(F, off) \
    *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(t1tab) + gulp_t1_byte(W1, (off), F.z, F.w))
        const uint2 P0 = DMX_T1(F0, 0u), P1 = DMX_T1(F1, o1), P2 = DMX_T1(F2, o2), P3 = DMX_T1(F3, o3);
#undef DMX_T1
        E0.x |= P0.x & 0x7F807F80u;
        E0.y |= P0.y;
        E1.x |= P1.x & 0x7F807F80u;
        E1.y |= P1.y;
        E2.x |= P2.x & 0x7F807F80u;
        E2.y |= P2.y;
        E3.x |= P3.x & 0x7F807F80u;
        E3.y |= P3.y;
        // tier 2: the lane's tier-1 escapes, their prefix over the wave
        const uint32_t d0 = (P0.x >> 15) & 7u, d1 = (P1.x >> 15) & 7u, d2 = (P2.x >> 15) & 7u;
        const uint32_t p1 = d0, p2 = p1 + d1, p3 = p2 + d2, cnt2 = p3 + ((P3.x >> 15) & 7u);
        const uint32_t inc1 = wave_scan_incl(cnt2);
        const uint32_t q1 = inc1 - cnt2;
        const uint32_t n2 = __builtin_amdgcn_readlane(inc1, 63);
        const uint32_t w2 = (n2 + 7u) >> 3;  // tier 2's words, 4 bits a tier-1 escape
        // The exact path takes a block with more tier-1 escapes than the
        // exchange holds (128 a wave, 8 a lane), a tail past the one word
        // each lane loaded, or streams past the block's end (a malformed
        // block the gate passes, whose tail lanes there loaded zeros: the
        // exact path reads memory, as a reader without an end bound does).
        // (the three uniform tests as one sign bit: every quantity here is
        // far below 2^31, so a difference that goes negative sets bit 31)
        const uint32_t past = (128u - n2) | (kGulpFixed + 64u - len) | (len - (kGulpFixed + w1 + w2));
        if (__builtin_expect((int32_t)past < 0 || __builtin_amdgcn_ballot_w64(cnt2 > 8u) != 0, 0)) {
            // exact lane-serial path over the streams in memory (tier 2's
            // length recounted there: the tail's tier-1 words may be short)
            const uint32_t* tp = data + block_start();
            const uint32_t* s1 = tp + kGulpFixed;
            const uint32_t* s2 = s1 + w1;
            uint32_t c2 = 0;
            for (uint32_t r = q0; r < q0 + cnt1; ++r) c2 += gulp_field(s1, r, 2) == 3u;
            const uint32_t i2 = wave_scan_incl(c2), b1 = i2 - c2;
            const uint32_t w2x = (__builtin_amdgcn_readlane(i2, 63) + 7u) >> 3;
            const uint32_t* s3 = s2 + w2x;
            const bool has_term = len > kGulpFixed + w1 + w2x;
            uint32_t c3 = 0;
            for (uint32_t r = b1; r < b1 + c2; ++r) c3 += gulp_field(s2, r, 4) == 15u;
            const uint32_t b2 = wave_scan_incl(c3) - c3;
            uint64_t elo = 0, ehi = 0;  // exponent byte of weight i: byte i & 7 of (i < 8 ? elo : ehi)
            uint32_t ra = q0, rb = b1, rc = b2;
            const uint32_t pw0 = palg[0], pw1 = palg[1];
#pragma unroll 1
            for (int i = 0; i < 16; ++i) {
                const uint32_t code = (T0 >> (2 * i)) & 3u;
                uint32_t e;
                if (code < 3u) {
                    e = (pw0 >> (8 * code)) & 0xFFu;
                } else {
                    const uint32_t c1 = gulp_field(s1, ra++, 2);
                    if (c1 < 3u) {
                        e = (pw1 >> (8 * c1)) & 0xFFu;
                    } else {
                        const uint32_t cc = gulp_field(s2, rb++, 4);
                        if (cc < 15u)
                            e = (palg[2 + (cc >> 2)] >> (8 * (cc & 3u))) & 0xFFu;
                        else
                            e = has_term ? gulp_field(s3, rc++, 8) : 0u;
                    }
                }
                const uint64_t v = (uint64_t)e << (8 * (i & 7));
                if (i < 8)
                    elo |= v;
                else
                    ehi |= v;
            }
            // exponent bytes 4g, 4g + 1 -> the pair E_g.x, 4g + 2, 4g + 3 -> E_g.y
            const uint32_t eb0 = (uint32_t)elo, eb1 = (uint32_t)(elo >> 32), eb2 = (uint32_t)ehi,
                           eb3 = (uint32_t)(ehi >> 32);
            E0 = make_uint2(__builtin_amdgcn_perm(0u, eb0, 0x0C010C00u) << 7, __builtin_amdgcn_perm(0u, eb0, 0x0C030C02u) << 7);
            E1 = make_uint2(__builtin_amdgcn_perm(0u, eb1, 0x0C010C00u) << 7, __builtin_amdgcn_perm(0u, eb1, 0x0C030C02u) << 7);
            E2 = make_uint2(__builtin_amdgcn_perm(0u, eb2, 0x0C010C00u) << 7, __builtin_amdgcn_perm(0u, eb2, 0x0C030C02u) << 7);
            E3 = make_uint2(__builtin_amdgcn_perm(0u, eb3, 0x0C010C00u) << 7, __builtin_amdgcn_perm(0u, eb3, 0x0C030C02u) << 7);
            if (M == 1) {
                __builtin_memcpy(&xa, xb, 16);
                __builtin_memcpy(&xc, xb + 512, 16);
            }
        } else {
            // lane j resolves tier-1 escapes 2j, 2j + 1 (codes ca, cb), code 15
            // escaping to the terminal
            uint32_t ea = pa, eb = pb;
            // (has_term, uniform and false unless the block has a terminal
            // stream, is tested first: then the per-lane tests are skipped)
            const bool has_term = len > kGulpFixed + w1 + w2;
            bool ta = false, tb = false;
            if (has_term) {
                ta = 2 * lane < n2 && ca == 15u;
                tb = 2 * lane + 1 < n2 && cb == 15u;
            }
            if (has_term && __builtin_amdgcn_ballot_w64(ta || tb) != 0) {
                const uint32_t nt = (uint32_t)ta + (uint32_t)tb;
                const uint32_t inc3 = wave_scan_incl(nt), q3 = inc3 - nt;
                // terminal byte r is byte r & 3 of its word r >> 2, tail word
                // w1 + w2 + (r >> 2)
                const uint32_t a3 = (q3 >> 2) << 2;
                const int at = (int)(a3 + 4u * (w1 + w2));
                uint32_t u0 = __builtin_amdgcn_ds_bpermute(at, s0.tail);
                uint32_t u1 = __builtin_amdgcn_ds_bpermute(at + 4, s0.tail);
                const uint32_t tstart = kGulpFixed + w1 + w2;
                if (__builtin_amdgcn_readlane(inc3, 63) > 4u * (len - tstart)) {
                    // a terminal shorter than its escapes (a malformed block
                    // the gate passes) loaded zeros past the block's end: its
                    // words from memory, as a reader without an end bound
                    // takes them (the wait also completes the stages in
                    // flight)
                    const uint32_t soff3 = (block_start() - base + tstart) * 4u;
                    asm volatile("buffer_load_dword %0, %2, %3, %4 offen\n\t"
                                 "buffer_load_dword %1, %2, %3, %4 offen offset:4\n\t"
                                 "s_waitcnt vmcnt(0)"
                                 : "=&v"(u0), "=&v"(u1)
                                 : "v"(a3), "s"(rsrc), "s"(soff3)
                                 : "memory");
                }
                const uint32_t tw = __builtin_amdgcn_alignbit(u1, u0, (q3 & 3u) << 3);
                if (ta) ea = tw & 0xFFu;
                if (tb) eb = ta ? (tw >> 8) & 0xFFu : tw & 0xFFu;
            }
            reinterpret_cast<uint16_t*>(x2)[lane] = (uint16_t)(ea | (eb << 8));
            __builtin_amdgcn_wave_barrier();
            // each lane's window of 8 exponent bytes from rank q1, placed by the
            // selector of (its tier-1 escapes before the group, the group's m1)
            const uint32_t kq = q1 >> 2;
            const uint32_t y0 = x2[kq], y1 = x2[kq + 1], y2 = x2[kq + 2];
            // the groups' selectors (by their tier-1 escapes before the group
            // and its mask m1); at M = 1 read with the activations in this
            // round trip (at M > 1 the registers are short: read at use)
#define DMX_SEL(P, off) sel2[((off) << 4) | ((P.x >> 3) & 15u)]
            uint2 sg0 = {}, sg1 = {}, sg2 = {}, sg3 = {};
            if (M == 1) {
                sg0 = DMX_SEL(P0, 0u);
                sg1 = DMX_SEL(P1, p1);
                sg2 = DMX_SEL(P2, p2);
                sg3 = DMX_SEL(P3, p3);
                __builtin_memcpy(&xa, xb, 16);
                __builtin_memcpy(&xc, xb + 512, 16);
                __builtin_amdgcn_sched_barrier(0);
            }
            const uint32_t wlo = __builtin_amdgcn_alignbit(y1, y0, (q1 & 3u) << 3);
            const uint32_t whi = __builtin_amdgcn_alignbit(y2, y1, (q1 & 3u) << 3);
#define DMX_T2(E, sv)                                     \
    {                                                     \
        const uint2 s = sv;                               \
        E.x |= __builtin_amdgcn_perm(whi, wlo, s.x) << 7; \
        E.y |= __builtin_amdgcn_perm(whi, wlo, s.y) << 7; \
    }
            DMX_T2(E0, M == 1 ? sg0 : DMX_SEL(P0, 0u))
            DMX_T2(E1, M == 1 ? sg1 : DMX_SEL(P1, p1))
            DMX_T2(E2, M == 1 ? sg2 : DMX_SEL(P2, p2))
            DMX_T2(E3, M == 1 ? sg3 : DMX_SEL(P3, p3))
#undef DMX_T2
#undef DMX_SEL
            __builtin_amdgcn_wave_barrier();
        }
        const uint32_t L0 = s0.lit.x, L1 = s0.lit.y, L2 = s0.lit.z, L3 = s0.lit.w;
        uint32_t wp[8];
        wp[0] = (__builtin_amdgcn_perm(L0, L0, 0x01010000) & keep) | (E0.x & ~keep);
        wp[1] = (__builtin_amdgcn_perm(L0, L0, 0x03030202) & keep) | (E0.y & ~keep);
        wp[2] = (__builtin_amdgcn_perm(L1, L1, 0x01010000) & keep) | (E1.x & ~keep);
        wp[3] = (__builtin_amdgcn_perm(L1, L1, 0x03030202) & keep) | (E1.y & ~keep);
        wp[4] = (__builtin_amdgcn_perm(L2, L2, 0x01010000) & keep) | (E2.x & ~keep);
        wp[5] = (__builtin_amdgcn_perm(L2, L2, 0x03030202) & keep) | (E2.y & ~keep);
        wp[6] = (__builtin_amdgcn_perm(L3, L3, 0x01010000) & keep) | (E3.x & ~keep);
        wp[7] = (__builtin_amdgcn_perm(L3, L3, 0x03030202) & keep) | (E3.y & ~keep);
        if constexpr (DEC) {
            // the lane's 16 weights: 32 bytes at weight 1024 blk + 16 lane
            uint4* d = reinterpret_cast<uint4*>(pick(g.out, ia)) + (uint64_t)c.blk * 128u + 2u * lane;
            d[0] = make_uint4(wp[0], wp[1], wp[2], wp[3]);
            d[1] = make_uint4(wp[4], wp[5], wp[6], wp[7]);
            sip_next<false>(sh, c, wk, sp);
            return;
        }
        if constexpr (QUAD) {
#pragma unroll
            for (int i = 0; i < 8; ++i) hout[i] = wp[i];
            quad_next(sh, cq, wk);
            return;
        }
        if (M == 1) {
            acc0 = dot2(wp[0], xa.x, acc0);
            acc1 = dot2(wp[1], xa.y, acc1);
            acc0 = dot2(wp[2], xa.z, acc0);
            acc1 = dot2(wp[3], xa.w, acc1);
            acc0 = dot2(wp[4], xc.x, acc0);
            acc1 = dot2(wp[5], xc.y, acc1);
            acc0 = dot2(wp[6], xc.z, acc0);
            acc1 = dot2(wp[7], xc.w, acc1);
        } else {
#pragma unroll
            for (int m = 0; m < MA; ++m) {
                uint4 ya, yc;
                __builtin_memcpy(&ya, xb + m * xrow, 16);
                __builtin_memcpy(&yc, xb + m * xrow + 512, 16);
                float a = acc[m];
                a = dot2(wp[0], ya.x, a);
                a = dot2(wp[1], ya.y, a);
                a = dot2(wp[2], ya.z, a);
                a = dot2(wp[3], ya.w, a);
                a = dot2(wp[4], yc.x, a);
                a = dot2(wp[5], yc.y, a);
                a = dot2(wp[6], yc.z, a);
                acc[m] = dot2(wp[7], yc.w, a);
            }
        }
        if (c.j + 1 == sh.seg_blocks) {
            if (M == 1) {
                const float s = wave_sum_dpp(acc0 + acc1);
                if (lane == 0) red[c.slot] = s;
                acc0 = acc1 = 0.0f;
            } else {
#pragma unroll
                for (int m = 0; m < MA; ++m) {
                    const float s = wave_sum_dpp(acc[m]);
                    if (lane == 0) red[c.slot * M + m] = s;
                    acc[m] = 0.0f;
                }
            }
        }
        sip_next<false>(sh, c, wk, sp);
    };
    const uint32_t my_units = wv < units ? (units - wv + W - 1) / W : 0;
    const uint32_t items = my_units * sh.seg_blocks * (QUAD ? 4 : 1);
    if constexpr (QUAD) {
        // a quad step (as in the sip kernel): the four rows' blocks of one
        // column block, stages A, B, C and D, each completed (nine loads
        // newer: the other three stages' three each), decoded and refilled at once with the
        // block four ahead; then the four rows meet the activation rows on
        // the matrix cores. One workgroup per CU (its registers), so no
        // workgroup priorities.
        uint32_t hq[4][8];
        const uint8_t* xq = reinterpret_cast<const uint8_t*>(xs) + (lane & 3u) * 2u * xrow + 64u * (lane >> 2);
        for (uint32_t k = 0; k < items; k += 4) {
            // the step's column block, phase and unit (shared by its four blocks)
            const uint32_t st_cb = cq.sp * sh.seg_blocks + cq.c, st_p = cq.p, st_row = 4 * cq.q;
            const uint32_t st_slot = st_row * sh.segs + cq.p * sh.psegs + cq.sp;
            const bool st_last = cq.c + 1 == sh.seg_blocks;
            GULP_WAIT(9, sA);
            process(sA, hq[0]);
            settle(hq[0]);
            uint2 oN = next_offsets();
            sA = gulp_load(rsrc, base, oN, ln);
            GULP_WAIT(9, sB);
            process(sB, hq[1]);
            settle(hq[1]);
            oN = next_offsets();
            sB = gulp_load(rsrc, base, oN, ln);
            GULP_WAIT(9, sC);
            process(sC, hq[2]);
            settle(hq[2]);
            oN = next_offsets();
            sC = gulp_load(rsrc, base, oN, ln);
            GULP_WAIT(9, sD);
            process(sD, hq[3]);
            settle(hq[3]);
            oN = next_offsets();
            sD = gulp_load(rsrc, base, oN, ln);
            if (PH)
                while (cur_phase < st_p) phase_advance();
            quad_transpose(hq, lane);
            quad_mfma<G>(dq, xq + st_cb * 2048u, 8u * xrow, hq);
            if (st_last) quad_unit_end<M, G>(dq, red, st_slot, sh.segs, st_row, nrows, lane);
        }
        // in flight now: the four stages, past the wave's work; they land
        // before the end
        GULP_WAIT(0, sD);
    } else {
    // Two workgroups share each SIMD, and its arbiter issues for the older
    // one's waves first: alone, the first workgroup finishes well before
    // the second, which then runs its last blocks without the other's
    // waves to hide its decode latency. The second one's waves issue at a
    // raised priority for their first three quarters of blocks, so both
    // finish nearer together (measured 2.5-3.4% faster on Qwen3-8B layers,
    // 1.4% on the 32B-class). sip streams near the read wall either way
    // and keeps the default.
    bool young = blockIdx.x >= sh.young_from;
    const uint32_t young_end = items - items / 4;
    if (young) __builtin_amdgcn_s_setprio(3);
    uint32_t k = 0;
    for (; k + 3 <= items; k += 3) {
        if (young && k >= young_end) {
            __builtin_amdgcn_s_setprio(0);
            young = false;
        }
        sC = gulp_load(rsrc, base, oC, ln);
        uint2 oN = next_offsets();
        GULP_WAIT(6, sA);
        process(sA, nullptr);
        sA = gulp_load(rsrc, base, oN, ln);
        oN = next_offsets();
        GULP_WAIT(6, sB);
        process(sB, nullptr);
        sB = gulp_load(rsrc, base, oN, ln);
        oC = next_offsets();
        GULP_WAIT(6, sC);
        process(sC, nullptr);
    }
    GULP_WAIT(3, sA);
    if (k < items) process(sA, nullptr);
    GULP_WAIT(0, sB);
    if (k + 1 < items) process(sB, nullptr);
    }
    if constexpr (DEC) return;  // every load has landed (the waits above)
    if (PH)
        while (cur_phase + 1 < sh.phases) phase_advance();
    __syncthreads();
    const void* bias = pick(g.bias, ia);
    void* out = pick(g.out, ia);
    const uint32_t rows_t = row_n - row_a;
    for (uint32_t i = threadIdx.x; i < nrows * sh.m; i += TH) {
        const uint32_t m = i / nrows, t = i - m * nrows;
        float sum = 0.0f;
        for (uint32_t k = 0; k < sh.segs; ++k) sum += red[(t * sh.segs + k) * M + m];
        if (bias) sum += load_elem(bias, sh.bias_dtype, lrow + t);
        store_elem(out, sh.out_dtype, (uint64_t)m * rows_t + lrow + t, sum);
    }
}

// ------------------------------------------------------ raw bf16 GEMV --
//
// drinkme's _gemv_narrow (src/drinkme/codec/radix_ops.py:177-249), the
// kernel of swap.NarrowLinear (src/drinkme/codec/swap.py:530-610): a raw
// row-major bf16 weight [R, C], no decoder, against M <= 8 activation rows.
// One workgroup of 256 threads per output row. Thread t takes the 8-column
// chunks t, t + 256, ... of the row and, per activation row, adds x * w
// over the chunk's columns in order with one fp32 fma each (16-byte loads
// where the row and x allow, else element loads: the same sums). The 256
// partials of a row are added in a fixed order (a DPP scan per wave, then
// the four waves in turn), the bias in fp32, one rounding at the store.
// Activation row m's arithmetic does not depend on M, so row m of an M-row
// call is the one-row call bit for bit; and since widening bf16 to fp32 is
// exact, a bf16 x gives the sums of its fp32 copy.
constexpr int kNarrowThreads = 256;

template <int M, bool VEC>
__global__ __launch_bounds__(kNarrowThreads) void k_gemv_narrow(const uint16_t* __restrict__ w, uint32_t cols,
                                                                const void* __restrict__ x, int x_dtype,
                                                                const void* bias, int bias_dtype, void* out,
                                                                int out_dtype, uint32_t rows) {
    __shared__ float red[M][kNarrowThreads / kWave];
    const uint32_t row = blockIdx.x;
    const uint16_t* wr = w + (uint64_t)row * cols;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    const uint32_t chunks = (cols + 7) / 8;
    for (uint32_t k = threadIdx.x; k < chunks; k += kNarrowThreads) {
        const uint32_t c0 = 8 * k, n = min(8u, cols - c0);
        float wf[8];
        if (VEC) {
            const uint4 v = *reinterpret_cast<const uint4*>(wr + c0);
            const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                wf[2 * e] = __uint_as_float(u[e] << 16);
                wf[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
            }
        } else {
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e) wf[e] = e < n ? bf16_bits_to_f32(wr[c0 + e]) : 0.0f;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const uint64_t xo = (uint64_t)m * cols + c0;
            float xf[8];
            if (VEC && x_dtype == DMX_BF16) {
                const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + xo);
                const uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    xf[2 * e] = __uint_as_float(u[e] << 16);
                    xf[2 * e + 1] = __uint_as_float(u[e] & 0xFFFF0000u);
                }
            } else if (VEC) {
                const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + xo);
                const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(x) + xo + 4);
                xf[0] = a.x, xf[1] = a.y, xf[2] = a.z, xf[3] = a.w;
                xf[4] = b.x, xf[5] = b.y, xf[6] = b.z, xf[7] = b.w;
            } else {
#pragma unroll
                for (uint32_t e = 0; e < 8; ++e) xf[e] = e < n ? load_elem(x, x_dtype, xo + e) : 0.0f;
            }
            float a = acc[m];
#pragma unroll
            for (uint32_t e = 0; e < 8; ++e)
                if (VEC || e < n) a = fmaf(xf[e], wf[e], a);
            acc[m] = a;
        }
    }
    const uint32_t wv = threadIdx.x / kWave;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float sum = wave_sum_dpp(acc[m]);
        if (lane_id() == 0) red[m][wv] = sum;
    }
    __syncthreads();
    if (threadIdx.x < (uint32_t)M) {
        const uint32_t m = threadIdx.x;
        float sum = 0.0f;
#pragma unroll
        for (int k = 0; k < kNarrowThreads / kWave; ++k) sum += red[m][k];
        if (bias) sum += load_elem(bias, bias_dtype, row);
        store_elem(out, out_dtype, (uint64_t)m * rows + row, sum);
    }
}

// ------------------------------------------------------ plain-read probe --
//
// A plain streaming read of `bytes` bytes of device memory: the ceiling a
// decode launch of the same bytes is measured against. The range is read
// as 1 KB rows, wave w of the grid's n taking rows w, w + n, w + 2n, ...,
// one non-temporal 16-byte load per lane per row (the payload loads'
// policy), one row in flight, through a buffer resource over exactly those
// bytes (a lane past the end reads 0 and fetches nothing). Of the layouts
// measured (rows interleaved or a contiguous run per wave; 768 or 1024
// threads; one, two or four rows in flight; one to eight workgroups per CU)
// this one, at two 1024-thread workgroups per CU, read the Qwen3-8B step's
// launches and a single 0.87 GB range fastest (6.3 and 7.0 TB/s). Each
// workgroup stores the XOR of every 32-bit word it read to
// sink[workgroup], so the reads cannot be dropped and a test can check
// them.
constexpr uint32_t kProbeThreads = 1024;

__global__ __launch_bounds__(kProbeThreads) void k_read_probe(const uint8_t* __restrict__ data, uint32_t bytes,
                                                               uint32_t* __restrict__ sink) {
    __shared__ uint32_t part[kProbeThreads / kWave];
    const i32x4 r = make_rsrc(data, bytes);
    const uint32_t lane = lane_id(), wv = wave_id();
    const uint32_t nw = gridDim.x * (kProbeThreads / kWave), gw = blockIdx.x * (kProbeThreads / kWave) + wv;
    const uint32_t rows = (bytes + 1023u) / 1024u;
    uint32_t acc = 0;
    for (uint32_t row = gw; row < rows; row += nw) {
        u32x4 a;
        asm volatile(
            "buffer_load_dwordx4 %0, %1, %2, 0 offen nt\n\t"
            "s_waitcnt vmcnt(0)"
            : "=&v"(a)
            : "v"(row * 1024u + 16u * lane), "s"(r)
            : "memory");
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
#pragma unroll
    for (int k = 32; k >= 1; k >>= 1) acc ^= __shfl_xor(acc, k, kWave);
    if (lane == 0) part[wv] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t x = 0;
#pragma unroll
        for (uint32_t k = 0; k < kProbeThreads / kWave; ++k) x ^= part[k];
        sink[blockIdx.x] = x;
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

// Raises the dynamic-LDS limit of a kernel family (its nk kernels) on the
// current device to at least `lds`. The limit only ever goes up, under one
// lock, so a concurrent caller cannot lower a limit another call's launch
// relies on. `preset` is the limit a kernel has before any opt-in.
enum LdsFamily { kFamSip, kFamGulp, kFamRaw, kFamDecodeSip, kFamDecodeGulp };
int raise_lds_limit(LdsFamily family, const void* const* kerns, int nk, size_t lds, size_t preset, const char* what,
                    char* err, size_t errn) {
    static std::mutex mu;
    static std::map<std::pair<int, int>, size_t> limit;  // (family, device) -> dynamic LDS allowed
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) dev = -1;
    std::lock_guard<std::mutex> lock(mu);
    size_t& cur = limit.try_emplace(std::make_pair((int)family, dev), preset).first->second;
    if (lds <= cur) return 0;
    for (int i = 0; i < nk; ++i) {
        const hipError_t e = hipFuncSetAttribute(kerns[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail_hip(err, errn, what, e);
    }
    cur = lds;
    return 0;
}

std::atomic<int> g_policy{DMX_POLICY_AUTO};

// The specialised kernels run under AUTO and MATRIX; MATRIX also puts
// gulp's 4-row verify in quad units.
bool fast_policy() {
    const int p = g_policy.load();
    return p == DMX_POLICY_AUTO || p == DMX_POLICY_MATRIX;
}
bool matrix_policy() { return g_policy.load() == DMX_POLICY_MATRIX; }

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

// The current device's CU count, cached per device (the plans deal rows
// to it).
int cu_count() {
    static std::mutex mu;
    static std::map<int, int> cached;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cached.find(dev);
    if (it != cached.end()) return it->second;
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached.emplace(dev, n);
    return n;
}

// Whether the sip kernel takes tensor t with this activation.
bool sip_eligible(const dmx_radix_tensor* t, const void* x, int x_dtype, uint32_t m) {
    return fast_policy() && m >= 1 && m <= 8 && x_dtype == DMX_BF16 && is_sip(t) &&
           t->block_size == 1024 &&
           t->cols % 1024 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

typedef void (*SipKernel)(const SipGroup, const uint16_t*, const SipShape);

// k_gemv_sip for M = 1, 2, 4, 8 (mi 0..3): one column phase (spanning tiles
// or not: kind 0, 1) or several (kind 2; tiles never span then)
SipKernel sip_kernel(int kind, int mi) {
    static const SipKernel table[3][4] = {
        {k_gemv_sip<false, 1, false>, k_gemv_sip<false, 2, false>, k_gemv_sip<false, 4, false>,
         k_gemv_sip<false, 8, false>},
        {k_gemv_sip<true, 1, false>, k_gemv_sip<true, 2, false>, k_gemv_sip<true, 4, false>,
         k_gemv_sip<true, 8, false>},
        {k_gemv_sip<false, 1, true>, k_gemv_sip<false, 2, true>, k_gemv_sip<false, 4, true>,
         k_gemv_sip<false, 8, true>}};
    return table[kind][mi];
}

// One launch of the sip kernel over n tensors of equal cols (already
// checked). Returns 2 when the group cannot run as one launch (a row tile
// taller than a tensor, or tables past the LDS), having launched nothing.
// The fast kernels address a tensor's directory with 32-bit byte offsets:
// tensors of 2^30 blocks or more (a trillion weights) run on the generic
// kernel.
bool fast_directory(const dmx_radix_tensor* t) {
    return (uint64_t)t->rows * ((t->cols + 1023) / 1024) < (1ull << 30);
}

int launch_sip(const dmx_radix_tensor* const* ts, uint32_t n, const void* x, uint32_t m, const void* const* bias,
               int bias_dtype, void* const* out, int out_dtype, hipStream_t stream, char* err, size_t errn) {
    if (n < 1 || n > (uint32_t)kGroupMax || m < 1 || m > 8) return 2;
    for (uint32_t i = 0; i < n; ++i)
        if (!fast_directory(ts[i])) return 2;
    const int mi = m == 1 ? 0 : m == 2 ? 1 : m <= 4 ? 2 : 3;
    const uint32_t M = 1u << mi;
    SipGroup g;
    SipShape sh;
    uint64_t total = 0;
    uint32_t min_rows = ts[0]->rows;
    for (uint32_t i = 0; i < (uint32_t)kGroupMax; ++i) {
        const dmx_radix_tensor* t = ts[i < n ? i : n - 1];
        g.data[i] = t->data;
        g.offsets[i] = t->offsets;
        g.palette[i] = t->palette;
        g.bias[i] = bias ? bias[i < n ? i : n - 1] : nullptr;
        g.out[i] = out[i < n ? i : n - 1];
        g.row0[i] = (uint32_t)total;
        if (i < n) {
            total += t->rows;
            min_rows = std::min(min_rows, t->rows);
        }
    }
    if (total >= (1ull << 31)) return 2;
    g.row0[kGroupMax] = (uint32_t)total;
    for (uint32_t i = n; i <= (uint32_t)kGroupMax; ++i) g.row0[i] = (uint32_t)total;
    sh.rows = (uint32_t)total;
    sh.cols = ts[0]->cols;
    sh.nb = sh.cols / 1024;
    sh.n = n;
    sh.m = m;
    sh.bias_dtype = bias_dtype;
    sh.out_dtype = out_dtype;
    const size_t fixed = kSipStaticLds;
    uint32_t grid = 0;
    size_t lds = 0;
    bool two = false;
    if (!plan_launch(sh, g.row0, n, min_rows, M, kSipWaves, kSipPerCu, sip_quad((int)M),
                     unit_end_cost(false, (int)M, false), fixed, true,
                     (uint32_t)cu_count(), grid, lds, two))
        return 2;
    {
        const void* kerns[12];
        for (int t = 0; t < 3; ++t)
            for (int i = 0; i < 4; ++i) kerns[4 * t + i] = reinterpret_cast<const void*>(sip_kernel(t, i));
        if (raise_lds_limit(kFamSip, kerns, 12, lds, 64 * 1024 - fixed, "sip kernel LDS opt-in", err, errn)) return 1;
    }
    hipLaunchKernelGGL(sip_kernel(sh.phases > 1 ? 2 : two ? 1 : 0, mi), dim3(grid), dim3(kSipThreads), lds, stream, g,
                       static_cast<const uint16_t*>(x), sh);
    return launch_check(err, errn, "sip gemv launch");
}

bool is_gulp(const dmx_radix_tensor* t) {
    return t->n_widths == 4 && t->widths[0] == 2 && t->widths[1] == 2 && t->widths[2] == 4 && t->widths[3] == 8;
}

bool gulp_eligible(const dmx_radix_tensor* t, const void* x, int x_dtype, uint32_t m) {
    return fast_policy() && m >= 1 && m <= 8 && x_dtype == DMX_BF16 && is_gulp(t) &&
           t->block_size == 1024 && t->cols % 1024 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

typedef void (*GulpKernel)(const SipGroup, const uint16_t*, const SipShape);

// waves: the plan's waves per workgroup (8 only unphased, M <= 4);
// matrix: the matrix policy's M = 4 (quad units)
GulpKernel gulp_kernel(bool phased, int mi, uint32_t waves = kSipWaves, bool matrix = false) {
    static const GulpKernel table[2][4] = {
        {k_gemv_gulp<1, false>, k_gemv_gulp<2, false>, k_gemv_gulp<4, false>, k_gemv_gulp<8, false>},
        {k_gemv_gulp<1, true>, k_gemv_gulp<2, true>, k_gemv_gulp<4, true>, k_gemv_gulp<8, true>}};
    static const GulpKernel table8[3] = {k_gemv_gulp<1, false, false, kGulpWaves3>,
                                         k_gemv_gulp<2, false, false, kGulpWaves3>,
                                         k_gemv_gulp<4, false, false, kGulpWaves3>};
    static const GulpKernel matrix4[2] = {k_gemv_gulp<4, false, false, kSipWaves, true>,
                                          k_gemv_gulp<4, true, false, kSipWaves, true>};
    if (matrix && mi == 2) return matrix4[phased ? 1 : 0];
    return waves == kGulpWaves3 && !phased && mi < 3 ? table8[mi] : table[phased ? 1 : 0][mi];
}

// One launch of the gulp kernel over n tensors of equal cols (already
// checked). Returns 2, having launched nothing, when it cannot take the
// group: a workgroup tile would span two tensors, or the LDS does not fit.
int launch_gulp(const dmx_radix_tensor* const* ts, uint32_t n, const void* x, uint32_t m, const void* const* bias,
                int bias_dtype, void* const* out, int out_dtype, hipStream_t stream, char* err, size_t errn) {
    if (n < 1 || n > (uint32_t)kGroupMax || m < 1 || m > 8) return 2;
    for (uint32_t i = 0; i < n; ++i)
        if (!fast_directory(ts[i])) return 2;
    const int mi = m == 1 ? 0 : m == 2 ? 1 : m <= 4 ? 2 : 3;
    const uint32_t M = 1u << mi;
    SipGroup g;
    SipShape sh;
    uint64_t total = 0;
    uint32_t min_rows = ts[0]->rows;
    for (uint32_t i = 0; i < (uint32_t)kGroupMax; ++i) {
        const dmx_radix_tensor* t = ts[i < n ? i : n - 1];
        g.data[i] = t->data;
        g.offsets[i] = t->offsets;
        g.palette[i] = t->palette;
        g.bias[i] = bias ? bias[i < n ? i : n - 1] : nullptr;
        g.out[i] = out[i < n ? i : n - 1];
        g.row0[i] = (uint32_t)total;
        if (i < n) {
            total += t->rows;
            min_rows = std::min(min_rows, t->rows);
        }
    }
    if (total >= (1ull << 31)) return 2;
    for (uint32_t i = n; i <= (uint32_t)kGroupMax; ++i) g.row0[i] = (uint32_t)total;
    sh.rows = (uint32_t)total;
    sh.cols = ts[0]->cols;
    sh.nb = sh.cols / 1024;
    sh.n = n;
    sh.m = m;
    sh.tbl2_lds = 0;
    sh.bias_dtype = bias_dtype;
    sh.out_dtype = out_dtype;
    const size_t fixed = kGulpStaticLds;
    uint32_t grid = 0;
    size_t lds = 0;
    bool two = false;
    const bool matrix = matrix_policy() && mi == 2;
    if (!plan_gulp(sh, g.row0, n, min_rows, M, (uint32_t)cu_count(), grid, lds, two, matrix)) return 2;
    {
        const void* kerns[13];
        for (int t = 0; t < 2; ++t)
            for (int i = 0; i < 4; ++i) kerns[4 * t + i] = reinterpret_cast<const void*>(gulp_kernel(t, i));
        for (int i = 0; i < 3; ++i) kerns[8 + i] = reinterpret_cast<const void*>(gulp_kernel(false, i, kGulpWaves3));
        for (int t = 0; t < 2; ++t) kerns[11 + t] = reinterpret_cast<const void*>(gulp_kernel(t, 2, kSipWaves, true));
        if (raise_lds_limit(kFamGulp, kerns, 13, lds, 64 * 1024 - fixed, "gulp kernel LDS opt-in", err, errn)) return 1;
    }
    if (sh.waves != kSipWaves && (sh.waves != kGulpWaves3 || sh.phases > 1 || mi == 3 || matrix)) return 2;
    hipLaunchKernelGGL(gulp_kernel(sh.phases > 1, mi, sh.waves, matrix), dim3(grid), dim3(64u * sh.waves), lds, stream,
                       g, static_cast<const uint16_t*>(x), sh);
    return launch_check(err, errn, "gulp gemv launch");
}

template <int M, bool RAW = false>
void launch_generic_m(const Desc& d, const void* x, int x_dtype, const void* bias, int bias_dtype, void* out,
                      int out_dtype, hipStream_t stream) {
    hipLaunchKernelGGL((k_gemv_generic<M, RAW>), dim3(d.rows), dim3(kGenThreads), 0, stream, d, x, x_dtype, bias,
                       bias_dtype, out, out_dtype);
}

int check_gemv_args(const void* x, int x_dtype, uint32_t m, const void* bias, int bias_dtype, const void* out,
                    int out_dtype, char* err, size_t errn) {
    if (!x || !out) return fail(err, errn, "null activation or output");
    if (m < 1 || m > 8) return fail(err, errn, "m outside 1..8");
    if ((x_dtype != DMX_BF16 && x_dtype != DMX_F32) || (out_dtype != DMX_BF16 && out_dtype != DMX_F32) ||
        (bias && bias_dtype != DMX_BF16 && bias_dtype != DMX_F32))
        return fail(err, errn, "dtype must be DMX_BF16 or DMX_F32");
    return 0;
}

int gemv_one(const dmx_radix_tensor* t, const Desc& d, const void* x, int x_dtype, uint32_t m, const void* bias,
             int bias_dtype, void* out, int out_dtype, hipStream_t s, char* err, size_t errn) {
    if (sip_eligible(t, x, x_dtype, m)) {
        const int rc = launch_sip(&t, 1, x, m, &bias, bias_dtype, &out, out_dtype, s, err, errn);
        if (rc != 2) return rc;
    }
    if (gulp_eligible(t, x, x_dtype, m)) {
        const int rc = launch_gulp(&t, 1, x, m, &bias, bias_dtype, &out, out_dtype, s, err, errn);
        if (rc != 2) return rc;
    }
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

template <int M>
void launch_narrow_m(bool vec, const uint16_t* w, uint32_t rows, uint32_t cols, const void* x, int x_dtype,
                     const void* bias, int bias_dtype, void* out, int out_dtype, hipStream_t s) {
    if (vec)
        hipLaunchKernelGGL((k_gemv_narrow<M, true>), dim3(rows), dim3(kNarrowThreads), 0, s, w, cols, x, x_dtype, bias,
                           bias_dtype, out, out_dtype, rows);
    else
        hipLaunchKernelGGL((k_gemv_narrow<M, false>), dim3(rows), dim3(kNarrowThreads), 0, s, w, cols, x, x_dtype,
                           bias, bias_dtype, out, out_dtype, rows);
}

}  // namespace

extern "C" int dmx_abi_version(void) { return DMX_ABI_VERSION; }

extern "C" uint64_t dmx_radix_pad_words(uint32_t block_size, const uint32_t* widths, uint32_t n_widths) {
    if (!widths) return 0;
    return pad_words_for(block_size, widths, n_widths);
}

extern "C" int dmx_radix_set_policy(int policy) {
    if (policy != DMX_POLICY_AUTO && policy != DMX_POLICY_GENERIC && policy != DMX_POLICY_MATRIX) return -1;
    return g_policy.exchange(policy);
}

// The decode of a whole-block sip or gulp tensor on its fast kernel's work
// split and decode (decode mode: the bits stored in place of the products).
// Returns 2, having launched nothing, when the tensor is not one of those
// (or would need column phases); the generic decoder then runs.
int launch_decode_fast(const dmx_radix_tensor* t, uint16_t* out, hipStream_t stream, char* err, size_t errn) {
    const bool sip = is_sip(t);
    const bool gulp = is_gulp(t);
    if (!fast_policy() || !(sip || gulp) || t->block_size != 1024 || t->cols % 1024 != 0 ||
        (reinterpret_cast<uintptr_t>(out) & 15u) != 0 || !fast_directory(t))
        return 2;
    SipGroup g;
    SipShape sh;
    for (uint32_t i = 0; i < (uint32_t)kGroupMax; ++i) {
        g.data[i] = t->data;
        g.offsets[i] = t->offsets;
        g.palette[i] = t->palette;
        g.bias[i] = nullptr;
        g.out[i] = out;
        g.row0[i] = i == 0 ? 0u : t->rows;
    }
    g.row0[kGroupMax] = t->rows;
    sh.rows = t->rows;
    sh.cols = t->cols;
    sh.nb = t->cols / 1024;
    sh.n = 1;
    sh.m = 1;
    sh.tbl2_lds = 0;
    sh.bias_dtype = sh.out_dtype = 0;
    const size_t fixed = sip ? kSipStaticLds : kGulpStaticLds;
    uint32_t grid = 0;
    size_t lds = 0;
    bool two = false;
    if (!plan_launch(sh, g.row0, 1, t->rows, 1, kSipWaves, kDecodePerCu, false, unit_end_cost(!sip, 1, true), fixed,
                     sip, (uint32_t)cu_count(),
                     grid, lds, two) ||
        sh.phases > 1)
        return 2;
    const void* kern = sip ? reinterpret_cast<const void*>(k_gemv_sip<false, 1, false, kModeDecode>)
                           : reinterpret_cast<const void*>(k_gemv_gulp<1, false, true>);
    if (raise_lds_limit(sip ? kFamDecodeSip : kFamDecodeGulp, &kern, 1, lds, 64 * 1024 - fixed,
                        "decode kernel LDS opt-in", err, errn))
        return 1;
    if (sip)
        hipLaunchKernelGGL((k_gemv_sip<false, 1, false, kModeDecode>), dim3(grid), dim3(kSipThreads), lds, stream, g,
                           static_cast<const uint16_t*>(nullptr), sh);
    else
        hipLaunchKernelGGL((k_gemv_gulp<1, false, true>), dim3(grid), dim3(kSipThreads), lds, stream, g,
                           static_cast<const uint16_t*>(nullptr), sh);
    return launch_check(err, errn, "decode launch");
}

extern "C" int dmx_radix_decode(const dmx_radix_tensor* t, uint16_t* out, void* stream, char* err, size_t errn) {
    Desc d;
    if (check_tensor(t, d, err, errn)) return 1;
    if (!out) return fail(err, errn, "null output");
    const int rc = launch_decode_fast(t, out, static_cast<hipStream_t>(stream), err, errn);
    if (rc != 2) return rc;
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
    if (check_gemv_args(x, x_dtype, m, bias, bias_dtype, out, out_dtype, err, errn)) return 1;
    return gemv_one(t, d, x, x_dtype, m, bias, bias_dtype, out, out_dtype, static_cast<hipStream_t>(stream), err,
                    errn);
}

extern "C" int dmx_radix_gemv_group(const dmx_radix_tensor* const* tensors, uint32_t n, const void* x, int x_dtype,
                                    uint32_t m, const void* const* bias, int bias_dtype, void* const* out,
                                    int out_dtype, void* stream, char* err, size_t errn) {
    if (!tensors || !out || n == 0) return fail(err, errn, "empty tensor group");
    Desc d[kGroupMax];
    bool all_sip = n <= (uint32_t)kGroupMax, all_gulp = all_sip;
    for (uint32_t i = 0; i < n; ++i) {
        Desc di;
        if (check_tensor(tensors[i], di, err, errn)) return 1;
        if (tensors[i]->cols != tensors[0]->cols) return fail(err, errn, "a tensor group must share cols (one activation)");
        if (check_gemv_args(x, x_dtype, m, bias ? bias[i] : nullptr, bias_dtype, out[i], out_dtype, err, errn))
            return 1;
        all_sip = all_sip && sip_eligible(tensors[i], x, x_dtype, m);
        all_gulp = all_gulp && gulp_eligible(tensors[i], x, x_dtype, m);
        if (i < (uint32_t)kGroupMax) d[i] = di;
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (all_sip) {
        const int rc = launch_sip(tensors, n, x, m, bias, bias_dtype, out, out_dtype, s, err, errn);
        if (rc != 2) return rc;
    }
    if (all_gulp) {
        const int rc = launch_gulp(tensors, n, x, m, bias, bias_dtype, out, out_dtype, s, err, errn);
        if (rc != 2) return rc;
    }
    for (uint32_t i = 0; i < n; ++i) {
        Desc di;
        if (i < (uint32_t)kGroupMax)
            di = d[i];
        else
            check_tensor(tensors[i], di, err, errn);
        if (gemv_one(tensors[i], di, x, x_dtype, m, bias ? bias[i] : nullptr, bias_dtype, out[i], out_dtype, s, err,
                     errn))
            return 1;
    }
    return 0;
}

extern "C" int dmx_gemv_narrow(const uint16_t* w, uint32_t rows, uint32_t cols, const void* x, int x_dtype,
                               uint32_t m, const void* bias, int bias_dtype, void* out, int out_dtype, void* stream,
                               char* err, size_t errn) {
    if (!w) return fail(err, errn, "null weight");
    if (rows == 0 || cols == 0) return fail(err, errn, "empty weight");
    if (rows >= (1u << 31)) return fail(err, errn, "too many rows");
    if (check_gemv_args(x, x_dtype, m, bias, bias_dtype, out, out_dtype, err, errn)) return 1;
    const bool vec = cols % 8 == 0 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (m) {
        case 1: launch_narrow_m<1>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 2: launch_narrow_m<2>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 3: launch_narrow_m<3>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 4: launch_narrow_m<4>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 5: launch_narrow_m<5>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 6: launch_narrow_m<6>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 7: launch_narrow_m<7>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        default: launch_narrow_m<8>(vec, w, rows, cols, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
    }
    return launch_check(err, errn, "narrow gemv launch");
}

// --------------------------------------------------------------- raw twin --

typedef void (*RawKernel)(const SipGroup, const uint16_t*, const SipShape);

// k_gemv_sip's raw instantiations: phased or not; M = 1, 2, 4, 8 (mi); at
// M = 4 and 8 the verify-row rule of the kernel mirrored (sip: quad units on
// the matrix cores; gulp: v_dot2 at M = 4, quad units with gulp's tiles at
// M = 8). At M = 1 and 2 the sip and gulp kernels do the same arithmetic,
// so one instantiation mirrors both.
constexpr int kRawKinds = 7;
RawKernel raw_kernel(bool phased, int kind) {
    static const RawKernel table[2][kRawKinds] = {
        {k_gemv_sip<false, 1, false, 1>, k_gemv_sip<false, 2, false, 1>, k_gemv_sip<false, 4, false, 1>,
         k_gemv_sip<false, 8, false, 1>, k_gemv_sip<false, 4, false, 2>, k_gemv_sip<false, 8, false, 2>,
         k_gemv_sip<false, 4, false, kModeTwinGulpMx>},
        {k_gemv_sip<false, 1, true, 1>, k_gemv_sip<false, 2, true, 1>, k_gemv_sip<false, 4, true, 1>,
         k_gemv_sip<false, 8, true, 1>, k_gemv_sip<false, 4, true, 2>, k_gemv_sip<false, 8, true, 2>,
         k_gemv_sip<false, 4, true, kModeTwinGulpMx>}};
    return table[phased ? 1 : 0][kind];
}
// (gulp's twin at M = 4 under the matrix policy: quad units, kind 6)
int raw_kind(int mi, bool gulp, bool matrix) { return gulp && matrix && mi == 2 ? 6 : gulp && mi >= 2 ? 2 + mi : mi; }

// The twin over the fast kernels' work split: the plan the mirrored kernel
// (sip, or gulp with `gulp`) makes for a tensor of this shape (its static
// LDS, matrix-core rule and waves), so every sum runs in that kernel's
// order. Returns 2, having launched nothing, when that kernel would not take
// the tensor either.
int launch_raw(const uint16_t* w, uint32_t rows, uint32_t cols, bool gulp, const void* x, uint32_t m,
               const void* bias, int bias_dtype, void* out, int out_dtype, hipStream_t stream, char* err,
               size_t errn) {
    if (m < 1 || m > 8) return 2;
    const int mi = m == 1 ? 0 : m == 2 ? 1 : m <= 4 ? 2 : 3;
    const uint32_t M = 1u << mi;
    SipGroup g;
    SipShape sh;
    for (uint32_t i = 0; i < (uint32_t)kGroupMax; ++i) {
        g.data[i] = reinterpret_cast<const uint32_t*>(w);
        g.offsets[i] = nullptr;
        g.palette[i] = nullptr;
        g.bias[i] = bias;
        g.out[i] = out;
        g.row0[i] = i == 0 ? 0u : rows;
    }
    g.row0[kGroupMax] = rows;
    sh.rows = rows;
    sh.cols = cols;
    sh.nb = cols / 1024;
    sh.n = 1;
    sh.m = m;
    sh.tbl2_lds = 0;
    sh.bias_dtype = bias_dtype;
    sh.out_dtype = out_dtype;
    const size_t fixed = gulp ? kGulpStaticLds : kSipStaticLds;
    const bool matrix = gulp && matrix_policy() && mi == 2;
    uint32_t grid = 0;
    size_t lds = 0;
    bool two = false;
    if (!plan_launch(sh, g.row0, 1, rows, M, kSipWaves, gulp ? gulp_per_cu((int)M, matrix) : kSipPerCu,
                     gulp ? gulp_quad((int)M, matrix) : sip_quad((int)M), unit_end_cost(gulp, (int)M, false, matrix),
                     fixed, !gulp, (uint32_t)cu_count(), grid, lds, two))
        return 2;
    if ((uint64_t)sh.rows_per_wg * cols * 2 >= (1ull << 31)) return 2;  // a tile's bytes within the buffer range
    {
        const void* kerns[2 * kRawKinds];  // (the raw kernels declare sip's static LDS)
        for (int t = 0; t < 2; ++t)
            for (int i = 0; i < kRawKinds; ++i) kerns[kRawKinds * t + i] = reinterpret_cast<const void*>(raw_kernel(t, i));
        if (raise_lds_limit(kFamRaw, kerns, 2 * kRawKinds, lds, 64 * 1024 - kSipStaticLds, "raw twin kernel LDS opt-in", err,
                            errn))
            return 1;
    }
    hipLaunchKernelGGL(raw_kernel(sh.phases > 1, raw_kind(mi, gulp, matrix)), dim3(grid), dim3(kSipThreads), lds, stream,
                       g, static_cast<const uint16_t*>(x), sh);
    return launch_check(err, errn, "raw twin gemv launch");
}

extern "C" int dmx_radix_gemv_twin(const uint16_t* w, uint32_t rows, uint32_t cols, uint32_t block_size,
                                   uint32_t n_widths, const uint32_t* widths, const void* x, int x_dtype, uint32_t m,
                                   const void* bias, int bias_dtype, void* out, int out_dtype, void* stream,
                                   char* err, size_t errn) {
    if (!w) return fail(err, errn, "null weight");
    if (rows == 0 || cols == 0) return fail(err, errn, "empty weight");
    if (block_size < 32 || block_size > 4096 || (block_size & (block_size - 1)))
        return fail(err, errn, "block_size must be a power of two from 32 through 4096");
    if (!widths || n_widths < 2 || n_widths > 8 || widths[n_widths - 1] != 8)
        return fail(err, errn, "radix needs 2..8 widths in 1..8, ending with the exponent width");
    if ((uint64_t)rows * ((cols + block_size - 1) / block_size) >= (1ull << 31)) return fail(err, errn, "too many blocks");
    if (check_gemv_args(x, x_dtype, m, bias, bias_dtype, out, out_dtype, err, errn)) return 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the kernel the compressed tensor of these widths would run (gemv_one)
    dmx_radix_tensor t = {};
    t.rows = rows;
    t.cols = cols;
    t.block_size = block_size;
    t.n_widths = n_widths;
    for (uint32_t j = 0; j < n_widths; ++j) t.widths[j] = widths[j];
    const bool fast = fast_policy() && m >= 1 && m <= 8 && x_dtype == DMX_BF16 &&
                      block_size == 1024 && cols % 1024 == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
    if (fast && (is_sip(&t) || is_gulp(&t))) {
        const int rc = launch_raw(w, rows, cols, is_gulp(&t), x, m, bias, bias_dtype, out, out_dtype, s, err, errn);
        if (rc != 2) return rc;
    }
    Desc d = {};
    d.data = reinterpret_cast<const uint32_t*>(w);
    d.rows = rows;
    d.cols = cols;
    d.block = block_size;
    d.nb = (cols + block_size - 1) / block_size;
    switch (m) {
        case 1: launch_generic_m<1, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 2: launch_generic_m<2, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 3: launch_generic_m<3, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 4: launch_generic_m<4, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 5: launch_generic_m<5, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 6: launch_generic_m<6, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        case 7: launch_generic_m<7, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
        default: launch_generic_m<8, true>(d, x, x_dtype, bias, bias_dtype, out, out_dtype, s); break;
    }
    return launch_check(err, errn, "raw twin generic gemv launch");
}

extern "C" int dmx_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t sink_words, void* stream,
                              char* err, size_t errn) {
    if (!data || !sink) return fail(err, errn, "null data or sink");
    if (bytes == 0 || bytes % 16 != 0) return fail(err, errn, "bytes must be a positive multiple of 16");
    if (bytes >= (1ull << 31)) return fail(err, errn, "a probe reads less than 2^31 bytes");
    if (sink_words == 0 || sink_words > 65535) return fail(err, errn, "sink_words (the workgroups) outside 1..65535");
    hipLaunchKernelGGL(k_read_probe, dim3(sink_words), dim3(kProbeThreads), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint8_t*>(data), (uint32_t)bytes, sink);
    return launch_check(err, errn, "read probe launch");
}
