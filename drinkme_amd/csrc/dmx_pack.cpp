// dmx_pack: drinkme's per-tensor pack step as a command, on host threads
// and without Python. It packs a bf16 weight the way pack_array_radix does
// (src/drinkme/codec/radix_pack.py:175-205: the native encoder, the CPU
// round trip, the raw fallback when radix would not compress) and writes the
// tensor file PackWriter.add writes (src/drinkme/codec/pack.py:509-520);
// and it reads one back through the load gates (pack.py:629-644).
//
//   dmx_pack encode [--profile sip|gulp|balanced] [--threads N] SRC.npy OUT.npz
//   dmx_pack decode NPZ OUT.npy
//   dmx_pack info NPZ
//   dmx_pack verify NPZ [SRC.npy]
//
// SRC.npy holds the bf16 bit patterns as uint16 ('<u2') [R, C]. Exit status
// 0 on success, 1 with the refusal on stderr.
#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "dmx_radix.h"

namespace {

int die(const std::string& msg) {
    std::fprintf(stderr, "dmx_pack: %s\n", msg.c_str());
    return 1;
}

double now() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// A C-order '<u2' [R, C] .npy, whole.
bool read_u16_npy(const char* path, std::vector<uint16_t>& out, uint64_t& R, uint64_t& C, std::string& err) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return err = std::string(path) + ": " + std::strerror(errno), false;
    unsigned char pre[12];
    if (std::fread(pre, 1, 10, f) != 10 || std::memcmp(pre, "\x93NUMPY", 6) != 0) {
        std::fclose(f);
        return err = std::string(path) + ": not a .npy array", false;
    }
    uint64_t hlen = pre[8] | (pre[9] << 8);
    if (pre[6] >= 2) {
        if (std::fread(pre + 10, 1, 2, f) != 2) {
            std::fclose(f);
            return err = std::string(path) + ": truncated .npy header", false;
        }
        hlen |= ((uint64_t)pre[10] << 16) | ((uint64_t)pre[11] << 24);
    }
    std::string h(hlen, '\0');
    if (std::fread(&h[0], 1, hlen, f) != hlen) {
        std::fclose(f);
        return err = std::string(path) + ": truncated .npy header", false;
    }
    if (h.find("'<u2'") == std::string::npos || h.find("'fortran_order': False") == std::string::npos) {
        std::fclose(f);
        return err = std::string(path) + ": need a C-order uint16 ('<u2') array of bf16 bit patterns", false;
    }
    const size_t s = h.find("'shape': (");
    if (s == std::string::npos ||
        std::sscanf(h.c_str() + s + 10, "%llu, %llu", (unsigned long long*)&R, (unsigned long long*)&C) != 2 ||
        R == 0 || C == 0) {
        std::fclose(f);
        return err = std::string(path) + ": need a nonempty 2-D array", false;
    }
    out.resize(R * C);
    const bool ok = std::fread(out.data(), 2, R * C, f) == R * C;
    std::fclose(f);
    if (!ok) return err = std::string(path) + ": truncated array", false;
    return true;
}

bool write_u16_npy(const char* path, const uint16_t* p, uint64_t R, uint64_t C, std::string& err) {
    std::string d = "{'descr': '<u2', 'fortran_order': False, 'shape': (" + std::to_string(R) + ", " +
                    std::to_string(C) + "), }";
    d.append((64 - (10 + d.size() + 1) % 64) % 64, ' ');
    d += '\n';
    FILE* f = std::fopen(path, "wb");
    if (!f) return err = std::string(path) + ": " + std::strerror(errno), false;
    const unsigned char pre[10] = {0x93, 'N', 'U', 'M', 'P', 'Y', 1, 0, (unsigned char)(d.size() & 0xFF),
                                   (unsigned char)(d.size() >> 8)};
    bool ok = std::fwrite(pre, 1, 10, f) == 10 && std::fwrite(d.data(), 1, d.size(), f) == d.size() &&
              std::fwrite(p, 2, R * C, f) == R * C;
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) err = std::string(path) + ": write failed";
    return ok;
}

uint32_t table_words(const uint32_t* w, uint32_t n) {
    uint32_t t = 0;
    for (uint32_t k = 0; k + 1 < n; ++k) t += ((1u << w[k]) + 2) / 4;
    return t;
}

// The palette, unpadded (the file's rx_palette), from the padded tables.
std::vector<uint8_t> palette_of(const std::vector<uint8_t>& tables, const uint32_t* w, uint32_t n) {
    std::vector<uint8_t> p;
    uint32_t at = 0;
    for (uint32_t k = 0; k + 1 < n; ++k) {
        const uint32_t m = (1u << w[k]) - 1;
        p.insert(p.end(), tables.begin() + at, tables.begin() + at + m);
        at += ((m + 3) / 4) * 4;
    }
    return p;
}

std::vector<uint8_t> tables_of(const std::vector<uint8_t>& palette, const uint32_t* w, uint32_t n) {
    std::vector<uint8_t> t(4 * table_words(w, n), 0);
    uint32_t at = 0, base = 0;
    for (uint32_t k = 0; k + 1 < n; ++k) {
        const uint32_t m = (1u << w[k]) - 1;
        std::memcpy(t.data() + at, palette.data() + base, m);
        at += ((m + 3) / 4) * 4;
        base += m;
    }
    return t;
}

int native(uint32_t op, void* src, uint64_t R, uint64_t C, const uint32_t* w, uint32_t nw, std::vector<uint8_t>& tables,
           std::vector<uint32_t>& offsets, std::vector<uint32_t>* data, uint64_t* result, std::string& err) {
    char e[512] = {};
    uint64_t res = 0;
    const uint64_t nb = (C + 1023) / 1024;
    const int st = dmx_radix_native(op, src, R, C, R, nb, 7, 8, w, nw, tables.data(), offsets.data(),
                                    data ? data->data() : nullptr, data ? data->size() : 0, 0, op == 2 ? R : 0, &res,
                                    e, sizeof e);
    if (st) err = std::string("native radix: ") + e;
    if (result) *result = res;
    return st;
}

int cmd_encode(int argc, char** argv) {
    std::string profile = "sip";
    int threads = 0;
    std::vector<const char*> pos;
    for (int i = 0; i < argc; ++i) {
        if (!std::strcmp(argv[i], "--profile") && i + 1 < argc)
            profile = argv[++i];
        else if (!std::strcmp(argv[i], "--threads") && i + 1 < argc)
            threads = std::atoi(argv[++i]);
        else
            pos.push_back(argv[i]);
    }
    if (pos.size() != 2) return die("usage: dmx_pack encode [--profile P] [--threads N] SRC.npy OUT.npz");
    uint32_t w[8], nw;
    if (profile == "sip") {
        w[0] = 3, w[1] = 8, nw = 2;
    } else if (profile == "balanced") {
        w[0] = 2, w[1] = 3, w[2] = 8, nw = 3;
    } else if (profile == "gulp") {
        w[0] = 2, w[1] = 2, w[2] = 4, w[3] = 8, nw = 4;
    } else {
        return die("unknown profile '" + profile + "' (sip | balanced | gulp)");
    }
    dmx_set_host_threads(threads);
    std::string err;
    std::vector<uint16_t> U;
    uint64_t R = 0, C = 0;
    if (!read_u16_npy(pos[0], U, R, C, err)) return die(err);
    const double t0 = now();
    const uint64_t nb = (C + 1023) / 1024;
    std::vector<uint8_t> tables(4 * table_words(w, nw), 0);
    std::vector<uint32_t> offsets(R * nb + 1, 0);
    uint64_t words = 0;
    if (native(0, U.data(), R, C, w, nw, tables, offsets, nullptr, &words, err)) return die(err);
    std::vector<uint32_t> data(words, 0);
    if (native(1, U.data(), R, C, w, nw, tables, offsets, &data, nullptr, err)) return die(err);
    // the CPU round trip (radix_pack.py:184-185: inside the encoder)
    std::vector<uint16_t> back(R * C);
    if (native(2, back.data(), R, C, w, nw, tables, offsets, &data, nullptr, err)) return die(err);
    if (back != U) return die("native radix: CPU round trip differs from the source bits");
    const double t1 = now();
    const std::vector<uint8_t> pal = palette_of(tables, w, nw);
    const uint64_t stored = pal.size() + 4 * offsets.size() + 4 * data.size();
    const uint64_t device = 4 * data.size() + 4 * offsets.size() + 4 * table_words(w, nw);
    dmx_pack_info info;
    std::memset(&info, 0, sizeof info);
    info.rows = R;
    info.cols = C;
    char e[1024] = {};
    int st;
    // the raw fallback (radix_pack.py:166-172): stored or device bytes reach the raw plane's
    if (std::max(stored, device) >= 2 * R * C) {
        info.codec = DMX_CODEC_RAW;
        info.bpw = 16.0;
        st = dmx_pack_write(pos[1], &info, nullptr, nullptr, nullptr, U.data(), e, sizeof e);
    } else {
        info.codec = DMX_CODEC_RADIX;
        info.block_size = 1024;
        info.n_widths = nw;
        for (uint32_t k = 0; k < nw; ++k) info.widths[k] = w[k];
        std::snprintf(info.profile, sizeof info.profile, "%s", profile.c_str());
        info.bpw = 8.0 * (double)stored / (double)(R * C);
        info.palette_len = pal.size();
        info.offsets_len = offsets.size();
        info.data_len = data.size();
        st = dmx_pack_write(pos[1], &info, pal.data(), offsets.data(), data.data(), nullptr, e, sizeof e);
    }
    if (st) return die(e);
    std::printf("%s: %llu x %llu, %s, bpw %.4f, %.2f s encode at %.2f GB/s bf16 in, %d threads\n", pos[1],
                (unsigned long long)R, (unsigned long long)C, info.codec == DMX_CODEC_RAW ? "raw" : profile.c_str(),
                info.bpw, t1 - t0, 2.0 * R * C / (t1 - t0) / 1e9, dmx_set_host_threads(threads));
    return 0;
}

// Reads NPZ through the gates; radix tensors decoded (with the decoder's
// exact-consumption checks) into bits.
int load(const char* path, dmx_pack_info& info, std::vector<uint16_t>& bits, std::string& err) {
    char e[1024] = {};
    if (dmx_pack_read(path, path, &info, nullptr, nullptr, nullptr, nullptr, e, sizeof e)) return err = e, 1;
    bits.assign(info.rows * info.cols, 0);
    if (info.codec == DMX_CODEC_RAW)
        return dmx_pack_read(path, path, &info, nullptr, nullptr, nullptr, bits.data(), e, sizeof e) ? (err = e, 1) : 0;
    std::vector<uint8_t> pal(info.palette_len);
    std::vector<uint32_t> offsets(info.offsets_len), data(info.data_len);
    if (dmx_pack_read(path, path, &info, pal.data(), offsets.data(), data.data(), nullptr, e, sizeof e))
        return err = e, 1;
    std::vector<uint8_t> tables = tables_of(pal, info.widths, info.n_widths);
    return native(2, bits.data(), info.rows, info.cols, info.widths, info.n_widths, tables, offsets, &data, nullptr,
                  err);
}

int cmd_decode(int argc, char** argv) {
    if (argc != 2) return die("usage: dmx_pack decode NPZ OUT.npy");
    dmx_pack_info info;
    std::vector<uint16_t> bits;
    std::string err;
    if (load(argv[0], info, bits, err)) return die(err);
    if (!write_u16_npy(argv[1], bits.data(), info.rows, info.cols, err)) return die(err);
    return 0;
}

int cmd_info(int argc, char** argv) {
    if (argc != 1) return die("usage: dmx_pack info NPZ");
    dmx_pack_info info;
    char e[1024] = {};
    if (dmx_pack_read(argv[0], argv[0], &info, nullptr, nullptr, nullptr, nullptr, e, sizeof e)) return die(e);
    if (info.codec == DMX_CODEC_RAW) {
        std::printf("{\"codec\": \"raw\", \"R\": %llu, \"C\": %llu, \"bpw\": %.6g}\n", (unsigned long long)info.rows,
                    (unsigned long long)info.cols, info.bpw);
    } else {
        std::string wl;
        for (uint32_t k = 0; k < info.n_widths; ++k) wl += (k ? ", " : "") + std::to_string(info.widths[k]);
        std::printf("{\"codec\": \"radix\", \"R\": %llu, \"C\": %llu, \"bpw\": %.6g, \"profile\": \"%s\", "
                    "\"widths\": [%s], \"block_size\": %u, \"palette\": %llu, \"offsets\": %llu, \"data_words\": %llu}\n",
                    (unsigned long long)info.rows, (unsigned long long)info.cols, info.bpw, info.profile, wl.c_str(),
                    info.block_size, (unsigned long long)info.palette_len, (unsigned long long)info.offsets_len,
                    (unsigned long long)info.data_len);
    }
    return 0;
}

int cmd_verify(int argc, char** argv) {
    if (argc != 1 && argc != 2) return die("usage: dmx_pack verify NPZ [SRC.npy]");
    dmx_pack_info info;
    std::vector<uint16_t> bits;
    std::string err;
    const double t0 = now();
    if (load(argv[0], info, bits, err)) return die(err);
    const double t1 = now();
    if (argc == 2) {
        std::vector<uint16_t> src;
        uint64_t R = 0, C = 0;
        if (!read_u16_npy(argv[1], src, R, C, err)) return die(err);
        if (R != info.rows || C != info.cols) return die("shape differs from the source");
        for (uint64_t i = 0; i < src.size(); ++i)
            if (src[i] != bits[i])
                return die("weight " + std::to_string(i) + " decodes to " + std::to_string(bits[i]) + ", source " +
                           std::to_string(src[i]));
    }
    std::printf("%s: ok (%llu x %llu%s), read + decode %.3f s\n", argv[0], (unsigned long long)info.rows,
                (unsigned long long)info.cols, argc == 2 ? ", equal to the source" : "", t1 - t0);
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 2) return die("usage: dmx_pack encode|decode|info|verify ...");
    const std::string cmd = argv[1];
    if (cmd == "encode") return cmd_encode(argc - 2, argv + 2);
    if (cmd == "decode") return cmd_decode(argc - 2, argv + 2);
    if (cmd == "info") return cmd_info(argc - 2, argv + 2);
    if (cmd == "verify") return cmd_verify(argc - 2, argv + 2);
    return die("unknown command '" + cmd + "' (encode | decode | info | verify)");
}
