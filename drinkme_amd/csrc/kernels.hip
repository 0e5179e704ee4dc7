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

#include <atomic>

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
// Layout: a workgroup of kSipWaves waves takes a tile of kSipWaves / S rows;
// the S waves of a row split its blocks into contiguous segments and their
// partial sums meet in LDS. Within a block, lane l owns weights 16l ..
// 16l + 15: its literals are the 16 bytes at word 4l (one 128-bit load) and
// its sixteen 3-bit tier-0 codes the 48 bits at bit 48l of the tier-0
// stream (two words). The activation sits in LDS; so does a per-workgroup
// table indexed by four codes (12 bits) that gives the exponent fields of
// the two bf16 pairs they belong to — E(c) << 7 | E(c') << 23, E of the
// escape code (7) = 0 — and, in the first word's low nibble, the four
// escape flags. A pair of weights is then one byte-permute of the literals
// merged (v_bfi) with its table word, and one v_dot2_f32_bf16 with the
// activation pair.
//
// Escaped weights: the main pass multiplies their literal with a zero
// exponent field (|w| < 2^-126, its product below every bound's absolute
// term for |x| < 2^96). Each lane then walks its own escapes: the rank of
// an escape in the terminal stream is the wave's exclusive prefix of
// escape counts (one DPP scan) plus the lane's running count; the
// terminal's words are staged in the wave's LDS slot, and the exact
// product x * w is added in fp32.

constexpr int kSipWaves = 16;
constexpr int kSipThreads = kSipWaves * kWave;
constexpr uint32_t kSipFixed = 256 + 96;  // literal plane + tier 0 words of a 1024-weight block
constexpr uint32_t kTableBytes = 4096 * 8;
constexpr uint32_t kTermWords = 256;  // the widest terminal stream of a block

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t w, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc,
                                           false);
}

struct SipArgs {
    const uint32_t* data;
    const uint32_t* offsets;
    const uint32_t* palette;
    const uint16_t* x;
    const void* bias;
    void* out;
    uint32_t rows, cols, nb, segs;
    int bias_dtype, out_dtype;
};

struct SipStage {
    uint4 lit;
    uint32_t t0lo, t0hi, term;
    uint32_t start, end;
};

__device__ __forceinline__ SipStage sip_load(const SipArgs& a, uint32_t blk, uint32_t lane) {
    SipStage s;
    s.start = a.offsets[blk];
    s.end = a.offsets[blk + 1];
    const uint32_t* base = a.data + s.start;
    __builtin_memcpy(&s.lit, base + 4 * lane, 16);
    const uint32_t w0 = (3 * lane) >> 1;
    s.t0lo = base[256 + w0];
    s.t0hi = base[256 + w0 + 1];
    const uint32_t nterm = s.end > s.start + kSipFixed ? s.end - s.start - kSipFixed : 0;
    s.term = lane < nterm ? base[kSipFixed + lane] : 0u;
    return s;
}

__global__ __launch_bounds__(kSipThreads) void k_gemv_sip(SipArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint2* tbl = reinterpret_cast<uint2*>(lds);
    uint16_t* xs = reinterpret_cast<uint16_t*>(lds + kTableBytes);
    uint32_t* term_all = reinterpret_cast<uint32_t*>(lds + kTableBytes + 2 * a.cols);
    float* red = reinterpret_cast<float*>(term_all + kSipWaves * kTermWords);

    // the exponent table of this tensor's palette: byte c of the two table
    // words is E(c), byte 7 the zero pad the escape code reads
    const uint32_t p0 = a.palette[0], p1 = a.palette[1];
    for (uint32_t g = threadIdx.x; g < 4096; g += kSipThreads) {
        uint32_t c0 = g & 7, c1 = (g >> 3) & 7, c2 = (g >> 6) & 7, c3 = (g >> 9) & 7;
        uint32_t e0 = __builtin_amdgcn_perm(p1, p0, c0) & 0xFF, e1 = __builtin_amdgcn_perm(p1, p0, c1) & 0xFF;
        uint32_t e2 = __builtin_amdgcn_perm(p1, p0, c2) & 0xFF, e3 = __builtin_amdgcn_perm(p1, p0, c3) & 0xFF;
        uint32_t flags = (c0 == 7) | ((c1 == 7) << 1) | ((c2 == 7) << 2) | ((c3 == 7) << 3);
        tbl[g] = make_uint2((e0 << 7) | (e1 << 23) | flags, (e2 << 7) | (e3 << 23));
    }
    for (uint32_t i = threadIdx.x; i < a.cols / 8; i += kSipThreads)
        reinterpret_cast<uint4*>(xs)[i] = reinterpret_cast<const uint4*>(a.x)[i];
    __syncthreads();

    const uint32_t wv = wave_id(), lane = lane_id();
    const uint32_t rows_per_tile = kSipWaves / a.segs;
    const uint32_t row = blockIdx.x * rows_per_tile + wv / a.segs;
    const uint32_t seg = wv % a.segs;
    const uint32_t b0 = seg * a.nb / a.segs, b1 = (seg + 1) * a.nb / a.segs;
    uint32_t* term = term_all + wv * kTermWords;
    const uint8_t* term_bytes = reinterpret_cast<const uint8_t*>(term);

    float acc0 = 0.0f, acc1 = 0.0f, acc_esc = 0.0f;
    if (row < a.rows && b0 < b1) {
        SipStage cur = sip_load(a, row * a.nb + b0, lane);
        for (uint32_t b = b0; b < b1; ++b) {
            SipStage nxt;
            if (b + 1 < b1) nxt = sip_load(a, row * a.nb + b + 1, lane);

            const uint64_t v = ((uint64_t)cur.t0hi << 32 | cur.t0lo) >> ((lane & 1) * 16);
            const uint32_t lo = (uint32_t)v;
            const uint2 E0 = tbl[lo & 0xFFF];
            const uint2 E1 = tbl[(lo >> 12) & 0xFFF];
            const uint2 E2 = tbl[(uint32_t)(v >> 24) & 0xFFF];
            const uint2 E3 = tbl[(uint32_t)(v >> 36) & 0xFFF];
            const uint16_t* xb = xs + b * 1024 + 16 * lane;
            uint4 xa, xc;
            __builtin_memcpy(&xa, xb, 16);
            __builtin_memcpy(&xc, xb + 8, 16);
            const uint32_t keep = 0x807F807Fu;  // sign + mantissa from the literal
            const uint32_t L0 = cur.lit.x, L1 = cur.lit.y, L2 = cur.lit.z, L3 = cur.lit.w;
            acc0 = dot2((__builtin_amdgcn_perm(L0, L0, 0x01010000) & keep) | (E0.x & ~keep), xa.x, acc0);
            acc1 = dot2((__builtin_amdgcn_perm(L0, L0, 0x03030202) & keep) | (E0.y & ~keep), xa.y, acc1);
            acc0 = dot2((__builtin_amdgcn_perm(L1, L1, 0x01010000) & keep) | (E1.x & ~keep), xa.z, acc0);
            acc1 = dot2((__builtin_amdgcn_perm(L1, L1, 0x03030202) & keep) | (E1.y & ~keep), xa.w, acc1);
            acc0 = dot2((__builtin_amdgcn_perm(L2, L2, 0x01010000) & keep) | (E2.x & ~keep), xc.x, acc0);
            acc1 = dot2((__builtin_amdgcn_perm(L2, L2, 0x03030202) & keep) | (E2.y & ~keep), xc.y, acc1);
            acc0 = dot2((__builtin_amdgcn_perm(L3, L3, 0x01010000) & keep) | (E3.x & ~keep), xc.z, acc0);
            acc1 = dot2((__builtin_amdgcn_perm(L3, L3, 0x03030202) & keep) | (E3.y & ~keep), xc.w, acc1);

            // escape flags, one nibble per group of four weights (byte j)
            const uint32_t m01 = __builtin_amdgcn_perm(E1.x, E0.x, 0x0C0C0400u);
            const uint32_t m23 = __builtin_amdgcn_perm(E3.x, E2.x, 0x0C0C0400u);
            uint32_t esc = __builtin_amdgcn_perm(m23, m01, 0x05040100u) & 0x0F0F0F0Fu;
            const uint32_t cnt = __builtin_popcount(esc);
            const uint32_t incl = wave_scan_incl(cnt);
            const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
            // the terminal is read only when the directory gives the block
            // words past its fixed streams (radix_kernel_gpu.py:96-98)
            if (total && cur.end > cur.start + kSipFixed) {
                const uint32_t need = (total + 3) >> 2;
                const uint32_t have = min(cur.end - cur.start - kSipFixed, (uint32_t)kWave);
                term[lane] = cur.term;
                for (uint32_t j = lane; j < need; j += kWave)
                    if (j >= have) term[j] = a.data[cur.start + kSipFixed + j];
                __builtin_amdgcn_wave_barrier();
                uint32_t q = incl - cnt;
                while (esc) {
                    const uint32_t p = __builtin_ctz(esc);
                    esc &= esc - 1;
                    const uint32_t grp = p >> 3, k = p & 3;
                    const uint32_t sel = (((grp & 1) << 2) | k) | 0x0C0C0C00u;
                    const uint32_t lb = (grp & 2) ? __builtin_amdgcn_perm(L3, L2, sel) : __builtin_amdgcn_perm(L1, L0, sel);
                    const uint32_t e = term_bytes[q++];
                    const uint32_t wbits = (__builtin_amdgcn_perm(0u, lb, 0x00000C0Cu) & ~0x7F800000u) | (e << 23);
                    const float xv = bf16_bits_to_f32(xb[4 * grp + k]);
                    acc_esc = fmaf(xv, __uint_as_float(wbits), acc_esc);
                }
                __builtin_amdgcn_wave_barrier();
            }
            cur = nxt;
        }
    }
    const float s = wave_sum(acc0 + acc1 + acc_esc);
    if (lane == 0) red[wv] = s;
    __syncthreads();
    if (threadIdx.x < rows_per_tile) {
        const uint32_t r = blockIdx.x * rows_per_tile + threadIdx.x;
        if (r < a.rows) {
            float sum = 0.0f;
            for (uint32_t k = 0; k < a.segs; ++k) sum += red[threadIdx.x * a.segs + k];
            if (a.bias) sum += load_elem(a.bias, a.bias_dtype, r);
            store_elem(a.out, a.out_dtype, r, sum);
        }
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
    SipArgs a;
    a.data = t->data;
    a.offsets = t->offsets;
    a.palette = t->palette;
    a.x = static_cast<const uint16_t*>(x);
    a.bias = bias;
    a.out = out;
    a.rows = t->rows;
    a.cols = t->cols;
    a.nb = t->cols / 1024;
    a.bias_dtype = bias_dtype;
    a.out_dtype = out_dtype;
    // waves per row: enough row segments that the grid holds ~16 waves per CU
    const uint64_t want = (uint64_t)cu_count() * 16;
    uint32_t segs = 1;
    while (segs < (uint32_t)kSipWaves && segs * 2 <= a.nb && (uint64_t)a.rows * segs < want) segs *= 2;
    a.segs = segs;
    const uint32_t rows_per_tile = kSipWaves / segs;
    const uint32_t grid = (a.rows + rows_per_tile - 1) / rows_per_tile;
    const size_t lds = kTableBytes + 2 * (size_t)a.cols + kSipWaves * kTermWords * 4 + kSipWaves * 4;
    static std::atomic<size_t> lds_opted{64 * 1024};
    if (lds > lds_opted.load()) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemv_sip),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail_hip(err, errn, "sip kernel LDS opt-in", e);
        lds_opted.store(lds);
    }
    hipLaunchKernelGGL(k_gemv_sip, dim3(grid), dim3(kSipThreads), lds, stream, a);
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
