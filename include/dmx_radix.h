/*
 * dmx_radix.h — the C ABI of drinkme_amd's MI355X (gfx950) radix codec
 * library, libdmx_radix.so.
 *
 * It replaces drinkme's fused radix decode + matmul path: the Triton module
 * codec/radix_ops.py that codec/swap.py binds through its one seam,
 * _bind_radix_ops (src/drinkme/codec/swap.py:60-65), plus the CPU codec's
 * single C entry point radix_native (src/drinkme/codec/radix_native.cpp:
 * 211-236). Every entry point below names the drinkme interface it stands
 * in for.
 *
 * Conventions (those of radix_native.cpp:211-236):
 *   - every entry point returns int: 0 on success, nonzero on a refusal;
 *     a refusal writes a NUL-terminated message into `err` (`errn` bytes);
 *   - every buffer is caller-owned: the library never allocates device
 *     memory and never frees; a device entry point only launches kernels
 *     on `stream` (a hipStream_t; NULL is the null stream) and returns
 *     without synchronising;
 *   - arguments are checked on the host before any launch, so a refusal
 *     launches nothing;
 *   - no per-load bounds in the kernels: `data` must carry at least
 *     dmx_radix_pad_words(block_size, widths) zero words after the payload
 *     (the reach pad, src/drinkme/codec/swap.py:84-95, :134-136) and the
 *     directory must have passed the descriptor gate
 *     (src/drinkme/codec/radix.py:174-238); then no read leaves the
 *     allocation, whatever the payload words hold.
 *
 * Formats: bf16 weights only; the radix stream layout of
 * docs/pack-format.md / src/drinkme/codec/radix.py:77-136 unchanged.
 */
#ifndef DMX_RADIX_H
#define DMX_RADIX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DMX_ABI_VERSION 1

/* element types of activations, biases and outputs */
#define DMX_BF16 0
#define DMX_F32 1

/* dmx_radix_set_policy */
#define DMX_POLICY_AUTO 0    /* the specialised kernels where they apply */
#define DMX_POLICY_GENERIC 1 /* the generic decoder for every tensor */
#define DMX_POLICY_MATRIX 2  /* as AUTO, with gulp's 3- and 4-row verify on the matrix cores too */

/* One radix tensor resident on the device: the runtime dict of
 * swap.to_device_radix (src/drinkme/codec/swap.py:80-161) as plain
 * pointers and scalars. */
typedef struct dmx_radix_tensor {
    const uint32_t* data;     /* rx_data: payload_words words, then pad_words zero words */
    const uint32_t* offsets;  /* rx_offsets: rows * ceil(cols / block_size) + 1 words */
    const uint32_t* palette;  /* rx_palette: each nonterminal tier's (1 << w) - 1 entries
                                 zero-padded to whole words, tiers concatenated
                                 (src/drinkme/codec/radix_pack.py:333-350) */
    const uint16_t* schedule; /* rx_schedule: one u16 per block for > 2 tiers, else NULL
                                 (dmx_radix_prepare writes it). Carried for drinkme's
                                 layout; no kernel here reads it (the gulp kernel finds
                                 its streams from each block's own counts), so it may be
                                 NULL */
    uint64_t payload_words;   /* NW */
    uint64_t pad_words;       /* zero words after the payload */
    uint32_t rows;            /* R */
    uint32_t cols;            /* C */
    uint32_t block_size;      /* B: power of two 32..4096 (the served format: 1024) */
    uint32_t n_widths;        /* tier count, terminal included: 2..8 */
    uint32_t widths[8];       /* tier widths; the last is 8 (the bf16 exponent) */
} dmx_radix_tensor;

/* DMX_ABI_VERSION of the loaded library. No drinkme counterpart (the
 * ctypes loader's version probe, src/drinkme/codec/radix_native.py:105-151). */
int dmx_abi_version(void);

/* The farthest word past a block's start any reader asks for:
 * block_word_bounds(B)[1] (src/drinkme/codec/radix.py:149-171); sip 608,
 * gulp 768 at B = 1024. 0 for invalid widths. */
uint64_t dmx_radix_pad_words(uint32_t block_size, const uint32_t* widths, uint32_t n_widths);

/* Replaces radix_native (src/drinkme/codec/radix_native.cpp:211-236) with
 * the same signature and meaning: op 0 plan (palette tables + directory,
 * *result = payload words), 1 encode, 2 decode rows [first, first + nrows)
 * into the pointer given (row `first` at its start), 3 validate the
 * palette tables. 1024-weight blocks; palettes per region of rg rows x cg
 * blocks. Runs on host threads (dmx_set_host_threads). */
int dmx_radix_native(uint32_t op, void* source_or_output, uint64_t rows, uint64_t cols, uint64_t rg,
                     uint64_t cg, uint32_t mant, uint32_t exponent, const uint32_t* widths, uint32_t count,
                     uint8_t* palettes, uint32_t* offsets, uint32_t* data, uint64_t words, uint64_t first,
                     uint64_t nrows, uint64_t* result, char* error, uint64_t error_size);

/* Host threads for dmx_radix_native and dmx_synth_bf16 (0 = all cores,
 * capped at 16). Returns the count now in force. No drinkme counterpart
 * (radix_native.py:220-259 threads in Python instead). */
int dmx_set_host_threads(int n);

/* Replaces radix_ops.decode_bits (src/drinkme/codec/radix_ops.py:418-427),
 * the _dense kernel (src/drinkme/codec/radix_kernel_gpu.py:614-636): every
 * block decoded once to the original u16 bit patterns, out [rows, cols]
 * (device, row-major). */
int dmx_radix_decode(const dmx_radix_tensor* t, uint16_t* out, void* stream, char* err, size_t errn);

/* Replaces radix_ops.prepare_schedule (src/drinkme/codec/radix_ops.py:
 * 341-348), the _prepare_schedule kernel (radix_kernel_gpu.py:44-66):
 * per block, byte (level - 1) = the word length of nonterminal tier
 * `level`'s stream, level >= 1. schedule: device, one u16 per block.
 * Refuses a two-tier tensor (sip has no schedule). */
int dmx_radix_prepare(const dmx_radix_tensor* t, uint16_t* schedule, void* stream, char* err, size_t errn);

/* Replaces radix_ops.gemv_fused / gemv / gemv_mc (src/drinkme/codec/
 * radix_ops.py:351-398) — the _gemv, _gemv_mc and _finish kernels
 * (radix_kernel_gpu.py:682-718, radix_ops.py:91-164).
 *   x     device [m, cols], x_dtype DMX_BF16 or DMX_F32, row stride cols;
 *   m     1..8 (ops.MC_MAX, src/drinkme/codec/ops.py:19);
 *   bias  device [rows] of bias_dtype, or NULL;
 *   out   device [m, rows] of out_dtype.
 * out = (x . W^T accumulated in fp32, + bias in fp32) rounded ONCE to
 * out_dtype (round to nearest even): gemv_fused's epilogue
 * (src/drinkme/codec/swap.py:284-300). m > 1 with bias NULL and DMX_F32
 * out is gemv_mc's fp32 [M, R]. */
int dmx_radix_gemv(const dmx_radix_tensor* t, const void* x, int x_dtype, uint32_t m, const void* bias,
                   int bias_dtype, void* out, int out_dtype, void* stream, char* err, size_t errn);

/* dmx_radix_gemv over n tensors that share one activation x (the q/k/v or
 * gate/up projections of a layer), as one launch where the kernels allow:
 * out[i] = dmx_radix_gemv(tensors[i], x, ..., bias ? bias[i] : NULL, out[i]).
 * Every tensor has the same cols; bias is NULL or n pointers (each may be
 * NULL). Each output is within the same bound of the float64 dot as
 * dmx_radix_gemv's, though its fp32 summation order may differ. No drinkme
 * counterpart: drinkme launches radix_ops.gemv_fused once per Linear
 * (src/drinkme/codec/swap.py:443-456); this is the grouped launch that
 * removes the per-launch cost from the decode step. Refuses (launching
 * nothing) on any tensor or argument dmx_radix_gemv refuses, or on unequal
 * cols. */
int dmx_radix_gemv_group(const dmx_radix_tensor* const* tensors, uint32_t n, const void* x, int x_dtype, uint32_t m,
                         const void* const* bias, int bias_dtype, void* const* out, int out_dtype, void* stream,
                         char* err, size_t errn);

/* Replaces radix_ops.gemv_narrow (src/drinkme/codec/radix_ops.py:401-415),
 * the _gemv_narrow kernel (radix_ops.py:177-249) that swap.NarrowLinear
 * runs (src/drinkme/codec/swap.py:530-610): a raw bf16 weight, no codec.
 *   w     device [rows, cols] bf16 bits, row-major;
 *   x     device [m, cols], x_dtype DMX_BF16 or DMX_F32, row stride cols;
 *   m     1..8;
 *   bias  device [rows] of bias_dtype, or NULL;
 *   out   device [m, rows] of out_dtype.
 * out = (x . w^T accumulated in fp32, + bias in fp32) rounded once. Row j
 * of an m-row call equals the one-row call on x's row j bit for bit, and a
 * bf16 x gives the same sums as its fp32 copy. */
int dmx_gemv_narrow(const uint16_t* w, uint32_t rows, uint32_t cols, const void* x, int x_dtype, uint32_t m,
                    const void* bias, int bias_dtype, void* out, int out_dtype, void* stream, char* err, size_t errn);

/* Replaces the raw twin of the GEMV calls: gemv_fused / gemv / gemv_mc over
 * a twin dict (src/drinkme/codec/radix_ops.py:252-255; swap.to_device_twin
 * swap.py:169-198, stock_linear swap.py:681-707), drinkme's kernels with
 * RAW=True (the decode replaced by a load of the raw weight,
 * radix_kernel_gpu.py:639-668). The kernel is the one dmx_radix_gemv runs
 * for a radix tensor of this shape, block size and widths (the twin dict's
 * widths are its compressed tensor's profile; sip's (3, 8) for a plain
 * Linear), with the weight read at each block's (row, column) in place of
 * the decode: the same work split and the same sums in the same order, so
 * the output equals dmx_radix_gemv's on the packed tensor bit for bit when
 * w is the packed tensor's source. w is 16-byte aligned for the fast
 * kernels (else the generic kernel's order applies).
 *   w        device [rows, cols] bf16 bits, row-major;
 *   widths   n_widths tier widths (2..8, the last 8), as the radix tensor's;
 *   x, m, bias, out as dmx_radix_gemv. */
int dmx_radix_gemv_twin(const uint16_t* w, uint32_t rows, uint32_t cols, uint32_t block_size, uint32_t n_widths,
                        const uint32_t* widths, const void* x, int x_dtype, uint32_t m, const void* bias,
                        int bias_dtype, void* out, int out_dtype, void* stream, char* err, size_t errn);

/* One tensor file of a drinkme pack (.npz: stored .npy members and a
 * `scalars` JSON blob; src/drinkme/codec/pack.py:509-520, :629-644). */
#define DMX_CODEC_RADIX 0 /* codec "radix": rx_palette, rx_offsets, rx_data */
#define DMX_CODEC_RAW 1   /* codec "raw": raw_bits */

typedef struct dmx_pack_info {
    uint32_t codec;       /* DMX_CODEC_RADIX or DMX_CODEC_RAW */
    uint32_t block_size;  /* radix: 1024 */
    uint64_t rows, cols;  /* R, C */
    uint32_t n_widths;    /* radix: tier count */
    uint32_t widths[8];
    char profile[16];     /* radix: "sip", "balanced" or "gulp" */
    double bpw;           /* the scalars' bpw */
    uint64_t palette_len; /* rx_palette entries (u8) */
    uint64_t offsets_len; /* rx_offsets entries (u32) */
    uint64_t data_len;    /* rx_data entries (u32) */
} dmx_pack_info;

/* Replaces pack._read_tensor (src/drinkme/codec/pack.py:629-644) for one
 * tensor file, without NumPy: the codec named by the scalars (:119-145),
 * R and C and the allocation cap off the ZIP directory (:164-207), then the
 * descriptor gate (validate_tensor :210-276 over radix.validate,
 * src/drinkme/codec/radix.py:174-238), each refusal in drinkme's words,
 * prefixed "pack tensor <name> (<codec>): ". Fills *info; then copies each
 * array whose buffer is non-NULL (host memory, sized from a first call
 * with NULL buffers: palette_len bytes, offsets_len and data_len words,
 * rows * cols u16 of raw_bits). Host threads: none. */
int dmx_pack_read(const char* path, const char* name, dmx_pack_info* info, uint8_t* palette, uint32_t* offsets,
                  uint32_t* data, uint16_t* raw_bits, char* err, size_t errn);

/* Replaces PackWriter.add's np.savez of one tensor (pack.py:509-520): a
 * ZIP of stored .npy members (ZIP64 where a member needs it) and the
 * scalars as json.dumps writes them, so np.load gives back the same arrays
 * and scalars string. Written to `path`.tmp, then renamed. */
int dmx_pack_write(const char* path, const dmx_pack_info* info, const uint8_t* palette, const uint32_t* offsets,
                   const uint32_t* data, const uint16_t* raw_bits, char* err, size_t errn);

/* Kernel choice for dmx_radix_gemv: DMX_POLICY_AUTO, DMX_POLICY_GENERIC
 * (an A/B switch like DRINKME_RADIX_DECODER, radix_ops.py:286-300) or
 * DMX_POLICY_MATRIX (AUTO's kernels, gulp's M = 3..4 verify rows in quad
 * units on the matrix cores, as M = 8 runs; AUTO keeps them on v_dot2,
 * measured faster there; the raw twin follows). No drinkme counterpart for
 * MATRIX: drinkme has one verify path. Process-global.
 * Returns the previous policy, or -1 for an unknown one. */
int dmx_radix_set_policy(int policy);

/* Seeded synthetic bf16 weights or activations for the workloads, no
 * drinkme counterpart: element i of stream (seed, stream) is a function of
 * i alone (counter-based), so any thread count writes the same bits.
 * dist 0: N(0, 1) * scale; dist 1: Student-t(nu = 4) / sqrt(2) * scale
 * (unit variance before the scale). float64 draw -> float32 (nearest) ->
 * bf16 (nearest even). Host memory. */
int dmx_synth_bf16(uint64_t seed, uint64_t stream, uint64_t count, double scale, uint32_t dist, uint16_t* out,
                   char* err, size_t errn);

/* A plain streaming read of `bytes` (a positive multiple of 16, below 2^31)
 * of device memory at `data`, with the payload loads' non-temporal 16-byte
 * reads: the ceiling that a decode launch of the same bytes is measured
 * against. No drinkme counterpart: a measurement probe. sink_words
 * workgroups of 1024 threads (1..65535) each read a contiguous share and
 * store the XOR of the 32-bit words they read to sink[workgroup], so the
 * XOR of sink[0 .. sink_words) is the XOR of every word of the range. */
int dmx_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t sink_words, void* stream, char* err,
                   size_t errn);

#ifdef __cplusplus
}
#endif

#endif /* DMX_RADIX_H */
