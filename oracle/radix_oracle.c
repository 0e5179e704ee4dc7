/*
 * ORACLE — test infrastructure only. A plain-C restatement of drinkme's radix
 * codec for bf16 weights, used as the checker by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg. The product
 * (drinkme_amd/) never links or calls it.
 *
 * What each function restates (paths relative to the drinkme source tree):
 *   orc_check_widths  src/drinkme/codec/radix.py:139-146 (_check_widths)
 *   orc_palette       src/drinkme/codec/radix.py:96-104 (histogram, stable
 *                     argsort of -hist, first `covered` entries);
 *                     radix_native.cpp:69-83 (count desc, ties exponent asc)
 *   orc_plan          src/drinkme/codec/radix_native.cpp:86-108 (per-block
 *                     word counts) == radix.py:107-121 (stream lengths)
 *   orc_encode        src/drinkme/codec/radix.py:105-120 (literal, tier
 *                     codes min(rank - base, escape), terminal exponents);
 *                     radix.py:50-61 (_put: little-endian fields in u32)
 *   orc_decode        src/drinkme/codec/radix.py:241-278 (decode) with
 *                     radix.py:64-74 (_get: 'truncated radix stream') and
 *                     the exact-consumption check ('trailing words')
 *   orc_padded_decode tests/test_radix_bounds.py:149-182 (padded_decode: the
 *                     device reader's model — zero words past the payload,
 *                     no consumption check, terminal read only if end > pos;
 *                     radix_kernel_gpu.py:96-98)
 *   orc_schedule      src/drinkme/codec/radix_pack.py:376-411 (schedule_np)
 *                     == tests/test_radix_pack.py:471-493
 *   orc_gemv_f64      bench/parity_common.py:231-251 (float64 dot and the
 *                     bound 2e-6 * |W|.|x| + 1e-7)
 *   orc_gemv_f32      src/drinkme/codec/swap.py:344-352 (the CPU route's
 *                     decode-then-matmul: fp32 accumulate, one rounding)
 *
 * Block size is a parameter (powers of two 32..4096, radix.py:88-89); the
 * served format fixes 1024. Only bf16 (7 mantissa bits + sign = 8-bit
 * literal, 8 exponent bits) is restated: fp8 is unserved.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MANT 7u
#define EXPW 8u

static int fail(char* err, size_t n, const char* msg) {
    if (err && n) {
        strncpy(err, msg, n - 1);
        err[n - 1] = 0;
    }
    return 1;
}

static uint64_t words_for(uint64_t count, uint32_t width) { return (count * width + 31) / 32; }

int orc_check_widths(const uint32_t* w, uint32_t nw, uint32_t* covered) {
    if (nw < 2 || nw > 8 || w[nw - 1] != EXPW) return 1;
    uint32_t cov = 0;
    for (uint32_t j = 0; j < nw; ++j)
        if (w[j] < 1 || w[j] > 8) return 1;
    for (uint32_t j = 0; j + 1 < nw; ++j) cov += (1u << w[j]) - 1;
    if (cov > 256) return 1;
    *covered = cov;
    return 0;
}

static uint32_t field_get(const uint32_t* s, uint64_t i, uint32_t w) {
    uint64_t bit = i * w;
    uint32_t sh = (uint32_t)(bit & 31);
    uint64_t k = bit >> 5;
    uint64_t v = s[k] >> sh;
    if (sh + w > 32) v |= (uint64_t)s[k + 1] << (32 - sh);
    return (uint32_t)(v & ((1u << w) - 1));
}

static void field_put(uint32_t* s, uint64_t i, uint32_t w, uint32_t v) {
    uint64_t bit = i * w;
    uint32_t sh = (uint32_t)(bit & 31);
    uint64_t k = bit >> 5;
    s[k] |= v << sh;
    if (sh + w > 32) s[k + 1] |= v >> (32 - sh);
}

/* palette[0..covered): exponents by count descending, ties by exponent
 * ascending (a stable argsort of -hist). */
int orc_palette(const uint16_t* bits, uint64_t R, uint64_t C, const uint32_t* widths, uint32_t nw,
                uint8_t* palette, char* err, size_t errn) {
    uint32_t covered;
    if (orc_check_widths(widths, nw, &covered)) return fail(err, errn, "invalid widths");
    uint64_t hist[256] = {0};
    for (uint64_t i = 0; i < R * C; ++i) hist[(bits[i] >> MANT) & 0xFF]++;
    int order[256];
    for (int e = 0; e < 256; ++e) order[e] = e;
    /* insertion sort: stable, so equal counts keep ascending exponents */
    for (int i = 1; i < 256; ++i) {
        int e = order[i], j = i - 1;
        while (j >= 0 && hist[order[j]] < hist[e]) {
            order[j + 1] = order[j];
            --j;
        }
        order[j + 1] = e;
    }
    for (uint32_t k = 0; k < covered; ++k) palette[k] = (uint8_t)order[k];
    return 0;
}

static void rank_table(const uint8_t* palette, uint32_t covered, uint16_t* rank_of) {
    for (int e = 0; e < 256; ++e) rank_of[e] = (uint16_t)covered;
    for (uint32_t k = 0; k < covered; ++k) rank_of[palette[k]] = (uint16_t)k;
}

/* offsets[0..R*NB]; returns 0 and the payload word count in *words. */
int orc_plan(const uint16_t* bits, uint64_t R, uint64_t C, uint32_t B, const uint32_t* widths,
             uint32_t nw, const uint8_t* palette, uint32_t* offsets, uint64_t* words, char* err,
             size_t errn) {
    uint32_t covered;
    if (orc_check_widths(widths, nw, &covered)) return fail(err, errn, "invalid widths");
    uint16_t rank_of[256];
    rank_table(palette, covered, rank_of);
    uint64_t nb = (C + B - 1) / B, total = 0;
    offsets[0] = 0;
    for (uint64_t r = 0; r < R; ++r) {
        for (uint64_t b = 0; b < nb; ++b) {
            uint64_t c0 = b * B, n = (C - c0 < B) ? C - c0 : B;
            uint64_t active = n, base = 0;
            total += words_for(n, MANT + 1);
            for (uint32_t j = 0; j + 1 < nw; ++j) {
                total += words_for(active, widths[j]);
                uint64_t esc = (1u << widths[j]) - 1, still = 0;
                for (uint64_t i = 0; i < n; ++i) {
                    uint32_t rk = rank_of[(bits[r * C + c0 + i] >> MANT) & 0xFF];
                    if (rk >= base + esc) still++;
                }
                active = still;
                base += esc;
            }
            total += words_for(active, EXPW);
            if (total > 0xFFFFFFFFull) return fail(err, errn, "radix payload exceeds the uint32 word directory");
            offsets[r * nb + b + 1] = (uint32_t)total;
        }
    }
    *words = total;
    return 0;
}

int orc_encode(const uint16_t* bits, uint64_t R, uint64_t C, uint32_t B, const uint32_t* widths,
               uint32_t nw, const uint8_t* palette, const uint32_t* offsets, uint32_t* data,
               uint64_t words, char* err, size_t errn) {
    uint32_t covered;
    if (orc_check_widths(widths, nw, &covered)) return fail(err, errn, "invalid widths");
    uint16_t rank_of[256];
    rank_table(palette, covered, rank_of);
    uint64_t nb = (C + B - 1) / B;
    memset(data, 0, words * 4);
    uint32_t* rk = malloc(sizeof(uint32_t) * B);
    uint32_t* ex = malloc(sizeof(uint32_t) * B);
    for (uint64_t r = 0; r < R; ++r) {
        for (uint64_t b = 0; b < nb; ++b) {
            uint64_t c0 = b * B, n = (C - c0 < B) ? C - c0 : B;
            uint32_t* s = data + offsets[r * nb + b];
            const uint16_t* src = bits + r * C + c0;
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t v = src[i];
                field_put(s, i, MANT + 1, (v & 0x7F) | ((v >> 15) << 7));
                ex[i] = (v >> MANT) & 0xFF;
                rk[i] = rank_of[ex[i]];
            }
            s += words_for(n, MANT + 1);
            uint64_t active = n;
            uint32_t base = 0;
            for (uint32_t j = 0; j + 1 < nw; ++j) {
                uint32_t w = widths[j], esc = (1u << w) - 1;
                uint64_t kept = 0;
                for (uint64_t i = 0; i < active; ++i) {
                    uint32_t code = rk[i] - base < esc ? rk[i] - base : esc;
                    field_put(s, i, w, code);
                    if (code == esc) {
                        rk[kept] = rk[i];
                        ex[kept] = ex[i];
                        kept++;
                    }
                }
                s += words_for(active, w);
                active = kept;
                base += esc;
            }
            for (uint64_t i = 0; i < active; ++i) field_put(s, i, EXPW, ex[i]);
            s += words_for(active, EXPW);
            if ((uint64_t)(s - data) != offsets[r * nb + b + 1]) {
                free(rk);
                free(ex);
                return fail(err, errn, "encode: block length differs from the plan");
            }
        }
    }
    free(rk);
    free(ex);
    return 0;
}

/* The CPU decoder with every check of radix.decode's block walk: a stream
 * reaching past the block's end is 'truncated radix stream', words left
 * over are 'radix block has trailing words'. The directory itself is
 * checked by the caller (radix.validate's restatement, in Python). */
int orc_decode(const uint8_t* palette, uint32_t covered, const uint32_t* offsets, const uint32_t* data,
               uint64_t words, uint64_t R, uint64_t C, uint32_t B, const uint32_t* widths, uint32_t nw,
               uint64_t first_row, uint64_t nrows, uint16_t* out, char* err, size_t errn) {
    uint32_t cov;
    if (orc_check_widths(widths, nw, &cov) || cov != covered) return fail(err, errn, "invalid widths");
    if (first_row > R || nrows > R - first_row) return fail(err, errn, "invalid decode range");
    uint64_t nb = (C + B - 1) / B;
    uint32_t* idx = malloc(sizeof(uint32_t) * B);
    int rc = 0;
    for (uint64_t r = first_row; r < first_row + nrows && !rc; ++r) {
        for (uint64_t b = 0; b < nb && !rc; ++b) {
            uint64_t blk = r * nb + b;
            uint64_t start = offsets[blk], end = offsets[blk + 1];
            if (end < start || end > words) {
                rc = fail(err, errn, "invalid radix block offsets");
                break;
            }
            const uint32_t* s = data + start;
            uint64_t len = end - start, pos = 0;
            uint64_t c0 = b * B, n = (C - c0 < B) ? C - c0 : B;
            uint16_t* dst = out + (r - first_row) * C + c0;
            if (words_for(n, MANT + 1) > len) {
                rc = fail(err, errn, "truncated radix stream");
                break;
            }
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t lit = field_get(s, i, MANT + 1);
                dst[i] = (uint16_t)((lit & 0x7F) | ((lit >> 7) << 15));
                idx[i] = (uint32_t)i;
            }
            pos = words_for(n, MANT + 1);
            uint64_t active = n;
            uint32_t base = 0;
            for (uint32_t j = 0; j + 1 < nw && !rc; ++j) {
                uint32_t w = widths[j], esc = (1u << w) - 1;
                if (pos + words_for(active, w) > len) {
                    rc = fail(err, errn, "truncated radix stream");
                    break;
                }
                uint64_t kept = 0;
                for (uint64_t i = 0; i < active; ++i) {
                    uint32_t code = field_get(s + pos, i, w);
                    if (code == esc) {
                        idx[kept++] = idx[i];
                    } else {
                        if (base + code >= covered) {
                            rc = fail(err, errn, "invalid radix palette index");
                            break;
                        }
                        dst[idx[i]] |= (uint16_t)(palette[base + code] << MANT);
                    }
                }
                pos += words_for(active, w);
                active = kept;
                base += esc;
            }
            if (rc) break;
            if (pos + words_for(active, EXPW) > len) {
                rc = fail(err, errn, "truncated radix stream");
                break;
            }
            for (uint64_t i = 0; i < active; ++i) dst[idx[i]] |= (uint16_t)(field_get(s + pos, i, EXPW) << MANT);
            pos += words_for(active, EXPW);
            if (pos != len) rc = fail(err, errn, "radix block has trailing words");
        }
    }
    free(idx);
    return rc;
}

/* A word read of the padded allocation: zero past the payload. */
static uint32_t padded_word(const uint32_t* data, uint64_t words, uint64_t k) { return k < words ? data[k] : 0; }

static uint32_t padded_field(const uint32_t* data, uint64_t words, uint64_t start, uint64_t i, uint32_t w) {
    uint64_t bit = i * w;
    uint32_t sh = (uint32_t)(bit & 31);
    uint64_t k = start + (bit >> 5);
    uint64_t v = padded_word(data, words, k) >> sh;
    if (sh + w > 32) v |= (uint64_t)padded_word(data, words, k + 1) << (32 - sh);
    return (uint32_t)(v & ((1u << w) - 1));
}

/* What the device readers produce over ANY directory (bounded by the
 * directory gate): radix.decode's walk with every word taken from the
 * padded allocation, no consumption check, and the terminal stream read
 * only when the block's end lies past the position the nonterminal tiers
 * reached. A palette index past `covered` reads the zero pad byte. */
int orc_padded_decode(const uint8_t* palette, uint32_t covered, const uint32_t* offsets, const uint32_t* data,
                      uint64_t words, uint64_t R, uint64_t C, uint32_t B, const uint32_t* widths, uint32_t nw,
                      uint16_t* out, char* err, size_t errn) {
    uint32_t cov;
    if (orc_check_widths(widths, nw, &cov) || cov != covered) return fail(err, errn, "invalid widths");
    uint64_t nb = (C + B - 1) / B;
    uint32_t* idx = malloc(sizeof(uint32_t) * B);
    for (uint64_t r = 0; r < R; ++r) {
        for (uint64_t b = 0; b < nb; ++b) {
            uint64_t blk = r * nb + b, start = offsets[blk], end = offsets[blk + 1];
            uint64_t c0 = b * B, n = (C - c0 < B) ? C - c0 : B;
            uint16_t* dst = out + r * C + c0;
            for (uint64_t i = 0; i < n; ++i) {
                uint32_t lit = padded_field(data, words, start, i, MANT + 1);
                dst[i] = (uint16_t)((lit & 0x7F) | ((lit >> 7) << 15));
                idx[i] = (uint32_t)i;
            }
            uint64_t pos = start + words_for(n, MANT + 1), active = n;
            uint32_t base = 0;
            for (uint32_t j = 0; j + 1 < nw; ++j) {
                uint32_t w = widths[j], esc = (1u << w) - 1;
                uint64_t kept = 0;
                for (uint64_t i = 0; i < active; ++i) {
                    uint32_t code = padded_field(data, words, pos, i, w);
                    if (code == esc) {
                        idx[kept++] = idx[i];
                    } else {
                        uint32_t e = base + code < covered ? palette[base + code] : 0;
                        dst[idx[i]] |= (uint16_t)(e << MANT);
                    }
                }
                pos += words_for(active, w);
                active = kept;
                base += esc;
            }
            if (end > pos)
                for (uint64_t i = 0; i < active; ++i)
                    dst[idx[i]] |= (uint16_t)(padded_field(data, words, pos, i, EXPW) << MANT);
        }
    }
    free(idx);
    return 0;
}

/* One u16 per block: byte (level - 1) = the word length of nonterminal tier
 * `level`'s stream, level >= 1. Escape counts read from the padded
 * allocation (zero past the payload). */
int orc_schedule(const uint32_t* offsets, const uint32_t* data, uint64_t words, uint64_t R, uint64_t C,
                 uint32_t B, const uint32_t* widths, uint32_t nw, uint16_t* sched, char* err, size_t errn) {
    uint32_t cov;
    if (orc_check_widths(widths, nw, &cov)) return fail(err, errn, "invalid widths");
    uint64_t nb = (C + B - 1) / B;
    for (uint64_t blk = 0; blk < R * nb; ++blk) {
        uint64_t n = C - (blk % nb) * B;
        if (n > B) n = B;
        uint64_t pos = offsets[blk] + words_for(n, MANT + 1), count = n;
        uint32_t header = 0;
        for (uint32_t level = 0; level + 1 < nw; ++level) {
            uint32_t w = widths[level];
            uint64_t len = words_for(count, w);
            if (level > 0) header |= (uint32_t)len << ((level - 1) * 8);
            if (level + 2 < nw) {
                uint64_t esc = 0;
                for (uint64_t i = 0; i < count; ++i) esc += padded_field(data, words, pos, i, w) == (1u << w) - 1;
                count = esc;
            }
            pos += len;
        }
        sched[blk] = (uint16_t)header;
    }
    return 0;
}

static double bf16_to_double(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

/* y[m, r] = sum_c W[r, c] x[m, c] in float64, and the cancellation-aware
 * bound 2e-6 * sum |W||x| + 1e-7. x is float32 [M, C]. */
void orc_gemv_f64(const uint16_t* bits, uint64_t R, uint64_t C, const float* x, uint64_t M, double* y,
                  double* bound) {
    for (uint64_t m = 0; m < M; ++m)
        for (uint64_t r = 0; r < R; ++r) {
            double s = 0, a = 0;
            const uint16_t* w = bits + r * C;
            const float* xm = x + m * C;
            for (uint64_t c = 0; c < C; ++c) {
                double wv = bf16_to_double(w[c]), xv = (double)xm[c];
                s += wv * xv;
                a += fabs(wv) * fabs(xv);
            }
            y[m * R + r] = s;
            bound[m * R + r] = 2e-6 * a + 1e-7;
        }
}

/* The CPU route's arithmetic: fp32 products accumulated in fp32 over the
 * decoded weight, the bias (if any) added in fp32 before the caller's one
 * rounding. */
void orc_gemv_f32(const uint16_t* bits, uint64_t R, uint64_t C, const float* x, uint64_t M,
                  const float* bias, float* y) {
    for (uint64_t m = 0; m < M; ++m)
        for (uint64_t r = 0; r < R; ++r) {
            float s = 0.0f;
            const uint16_t* w = bits + r * C;
            const float* xm = x + m * C;
            for (uint64_t c = 0; c < C; ++c) {
                uint32_t u = (uint32_t)w[c] << 16;
                float wv;
                memcpy(&wv, &u, 4);
                s += wv * xm[c];
            }
            y[m * R + r] = bias ? s + bias[r] : s;
        }
}
