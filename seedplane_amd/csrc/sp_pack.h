// Host packer: canonical weight layouts (seedplane_hip.h, SP_FMT_*) -> the tiled HBM layout the kernels read.
//
// A matrix [rows][K] is cut into 16-row groups; each group into k-tiles of KT columns (F16: 32, Q8: 64, Q4: 128).
// Tiles are stored row-group-major, k-tile-minor, 1024 code bytes each, so one row group streams contiguously.
// Inside a tile, lane l (0..63) of the consuming wave reads bytes [16l, 16l + 16): row r = l % 16, k-subset
// g = l / 16, i.e. exactly the B operand of a 16x16x32 MFMA per quant block:
//   F16: 8 fp16   w[r][32kt + 8g + i]                                    (i = 0..7)
//   Q8 : 8 int8   c[r][64kt + 8g + i]      then 8 int8 c[r][64kt + 32 + 8g + i]   (block 2kt, block 2kt+1)
//   Q4 : 4 dwords, dword s = 8 nibbles c[r][128kt + 32s + 8g + i], code i at nibble (i/2) + 4*(i%2)
// Per-tile side data (fp16), row r's entries contiguous so one lane load fetches them:
//   Q8 : scale[r][blk]                 (16 x 2)      64 bytes per tile
//   Q4 : (scale, zero)[r][group s]     (16 x 4 x 2)  256 bytes per tile
// Rows are zero-padded to a multiple of 16.  With `pair_halves` (SwiGLU gate_up [2I][K]) the row groups are
// reordered gate(16u..16u+15), up(16u..16u+15), gate(16u+16..), ... so one unit of 32 rows holds the gate and up
// rows of the same 16 outputs.
#pragma once
#include <cstdint>
#include <cstring>
#include <algorithm>
#include <stdexcept>
#include <thread>
#include <vector>

namespace sp {

struct Packed {
    int fmt = 0, rows = 0, cols = 0, rows_pad = 0, nkt = 0;
    std::vector<uint8_t> codes;   // rows_pad/16 * nkt * 1024
    std::vector<uint16_t> sz;     // per-tile side data (fp16 bits)
};

inline int kt_of(int fmt) { return fmt == 1 ? 32 : fmt == 2 ? 64 : 128; }

// canonical row of packed row p
inline int src_row(int p, int rows, bool pair_halves) {
    if (!pair_halves) return p;
    const int half_rows = rows / 2;
    const int rg = p / 16, r = p % 16, u = rg / 2, h = rg % 2;
    return h * half_rows + 16 * u + r;
}

inline Packed pack_matrix(int fmt, int rows, int cols, const void *data, const void *scales, const void *zeros,
                          bool pair_halves) {
    if (fmt != 1 && fmt != 2 && fmt != 3) throw std::invalid_argument("unsupported weight format");
    const int KT = kt_of(fmt);
    if (rows <= 0 || cols <= 0 || cols % KT) throw std::invalid_argument("matrix columns must be a positive multiple of the k-tile (F16 32, Q8 64, Q4 128)");
    if (pair_halves && (rows % 32)) throw std::invalid_argument("gate_up rows must be 2 * a multiple of 16");
    if (!data || (fmt >= 2 && !scales) || (fmt == 3 && !zeros)) throw std::invalid_argument("missing weight buffers");
    Packed p;
    p.fmt = fmt; p.rows = rows; p.cols = cols;
    p.rows_pad = (rows + 15) / 16 * 16; p.nkt = cols / KT;
    const int ngroups = p.rows_pad / 16;
    p.codes.assign((size_t)ngroups * p.nkt * 1024, 0);
    if (fmt == 2) p.sz.assign((size_t)ngroups * p.nkt * 32, 0);
    if (fmt == 3) p.sz.assign((size_t)ngroups * p.nkt * 128, 0);
    const int nblk = cols / 32;
    auto do_group = [&](int rg) {
        for (int r = 0; r < 16; ++r) {
            const int prow = rg * 16 + r;
            if (prow >= rows) continue;
            const int srow = src_row(prow, rows, pair_halves);
            for (int kt = 0; kt < p.nkt; ++kt) {
                const size_t tile = (size_t)rg * p.nkt + kt;
                uint8_t *t = p.codes.data() + tile * 1024;
                for (int g = 0; g < 4; ++g) {
                    uint8_t *lane = t + (size_t)(g * 16 + r) * 16;
                    if (fmt == 1) {
                        const uint16_t *w = (const uint16_t *)data + (size_t)srow * cols;
                        std::memcpy(lane, w + kt * 32 + 8 * g, 16);
                    } else if (fmt == 2) {
                        const int8_t *c = (const int8_t *)data + (size_t)srow * cols;
                        std::memcpy(lane, c + kt * 64 + 8 * g, 8);
                        std::memcpy(lane + 8, c + kt * 64 + 32 + 8 * g, 8);
                    } else {
                        const uint8_t *c = (const uint8_t *)data + (size_t)srow * (cols / 2);
                        for (int s = 0; s < 4; ++s) {
                            uint32_t d = 0;
                            for (int i = 0; i < 8; ++i) {
                                const int k = kt * 128 + 32 * s + 8 * g + i;
                                const uint32_t code = (c[k >> 1] >> ((k & 1) * 4)) & 15u;
                                d |= code << (4 * ((i >> 1) + 4 * (i & 1)));
                            }
                            std::memcpy(lane + 4 * s, &d, 4);
                        }
                    }
                }
                if (fmt == 2) {
                    const uint16_t *s = (const uint16_t *)scales + (size_t)srow * nblk;
                    for (int b = 0; b < 2; ++b) p.sz[tile * 32 + r * 2 + b] = s[kt * 2 + b];
                } else if (fmt == 3) {
                    const uint16_t *s = (const uint16_t *)scales + (size_t)srow * nblk;
                    const uint16_t *z = (const uint16_t *)zeros + (size_t)srow * nblk;
                    for (int gi = 0; gi < 4; ++gi) {
                        p.sz[tile * 128 + (r * 4 + gi) * 2] = s[kt * 4 + gi];
                        p.sz[tile * 128 + (r * 4 + gi) * 2 + 1] = z[kt * 4 + gi];
                    }
                }
            }
        }
    };
    // row groups are independent: spread them over the host cores
    const int nth = std::max(1, std::min<int>((int)std::thread::hardware_concurrency(), 16));
    if (nth == 1 || ngroups < 64) {
        for (int rg = 0; rg < ngroups; ++rg) do_group(rg);
    } else {
        std::vector<std::thread> pool;
        for (int t = 0; t < nth; ++t)
            pool.emplace_back([&, t] { for (int rg = t; rg < ngroups; rg += nth) do_group(rg); });
        for (auto &th : pool) th.join();
    }
    return p;
}

}  // namespace sp
