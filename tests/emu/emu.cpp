// Host emulation of the gfx950 matvec kernel (siphon_amd/csrc/matvec.h).
// TEST INFRASTRUCTURE ONLY: it compiles the product's own layout, repack and
// per-unit decode code (formats.h, unit.h) for the CPU and replays the
// kernel's tile / lane / step loops and its xor-butterfly reduction order,
// so indexing and decoding can be checked against the oracle without a GPU.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "../../siphon_amd/csrc/formats.h"
#include "../../siphon_amd/csrc/unit.h"

using namespace sihip;

static int64_t lds_col(uint32_t pair, int64_t n) {
    int64_t b = pair == T_Q8_K ? n + (n / 256) * 36 : pair == T_Q8_0 ? n + (n / 32) * 8 : n * 2;
    return (b + 15) & ~(int64_t)15;
}

// Stage one pair-format activation row (reference block layout) into the
// LDS column layout the kernel uses.
static void stage(uint32_t pair, int64_t n, const uint8_t *xq, uint8_t *col) {
    if (pair == T_Q8_K) {
        const int64_t nb = n / 256;
        for (int64_t b = 0; b < nb; b++) {
            memcpy(col + n + b * 4, xq + b * 292, 4);
            for (int k = 0; k < 8; k++)
                memcpy(col + q8k_lds_unit((uint32_t)nb, (uint32_t)b, (uint32_t)k),
                       xq + b * 292 + 4 + 32 * k, 32);
            memcpy(col + n + nb * 4 + b * 32, xq + b * 292 + 260, 32);
        }
    } else if (pair == T_Q8_0) {
        const int64_t nb = n / 32;
        for (int64_t b = 0; b < nb; b++) {
            const uint8_t *s = xq + b * 34;
            const float d = half_to_float((uint32_t)s[0] | ((uint32_t)s[1] << 8));
            int sum = 0;
            for (int k = 0; k < 32; k++) sum += (int8_t)s[2 + k];
            memcpy(col + b * 32, s + 2, 32);
            memcpy(col + n + b * 4, &d, 4);
            memcpy(col + n + nb * 4 + b * 4, &sum, 4);
        }
    } else {
        memcpy(col, xq, (size_t)n * 2);
    }
}

// spr: rounds per column slice (slice_rounds); the partial sums of the
// slices are added in slice order, starting from 0.0f, as the kernel's
// reduction does; one slice (spr == L.S) is the row's value itself.
template <uint32_t FMT>
static void run(const Layout &L, const uint8_t *W, const uint8_t *lds, int64_t cb, int64_t spr,
                float *y) {
    Planes P;
    for (int p = 0; p < 4; p++) P.p[p] = W + L.plane_off[p];
    for (int64_t tile = 0; tile < L.ntiles; tile++) {
        for (int r = 0; r < L.R; r++) {
            const int64_t row = tile * L.R + r;
            float yrow = 0.0f;
            for (int64_t s0 = 0; s0 < L.S; s0 += spr) {
            const int64_t s1 = s0 + spr < L.S ? s0 + spr : L.S;
            std::vector<float> v(L.G, 0.0f);
            for (int g = 0; g < L.G; g++) {
                const uint32_t lane = (uint32_t)(r * L.G + g);
                float acc[1] = {0.0f};
                // the rounds of the slice; a padding slot (column past the
                // row, last round only) re-reads the row's last real column
                // of that round and its contribution is discarded
                const int64_t glast = L.ncols - 1 - (L.S - 1) * L.G;
                const uint32_t lane_last =
                    (uint32_t)(r * L.G + (g < glast ? g : glast));
                for (int64_t s = s0; s < s1; s++) {
                    int64_t col = s * L.G + g;
                    const bool pad = col > L.ncols - 1;
                    if (pad) col = L.ncols - 1;
                    const uint32_t ln = s == L.S - 1 ? lane_last : lane;
                    const uint32_t rec = (uint32_t)((tile * L.S + s) * 64);
                    const float keep = acc[0];
                    if constexpr (is_kquant(FMT)) {
                        KRaw raw;
                        load_kblock<FMT>(P, rec * 8u + ln, rec + ln, raw);
                        compute_kblock<FMT, 1>(lds, (uint32_t)cb, (uint32_t)L.n_in, (uint32_t)col,
                                               raw, acc);
                    } else {
                        Raw raw;
                        load_unit<FMT>(P, rec + ln, raw);
                        compute_unit<FMT, 1>(lds, (uint32_t)cb, (uint32_t)L.n_in, (uint32_t)col,
                                             raw, acc);
                    }
                    if (pad) acc[0] = keep;
                }
                v[g] = acc[0];
            }
            // the kernel's group_sum: step k adds the value of reduce_partner(lane, k)
            for (int k = 0; (1 << k) < L.G; k++) {
                std::vector<float> nv(L.G);
                for (int g = 0; g < L.G; g++) nv[g] = v[g] + v[reduce_partner(g, k)];
                v = nv;
            }
            yrow = spr >= L.S ? v[0] : yrow + v[0];
            }
            if (row < L.n_out) y[row] = yrow;
        }
    }
}

extern "C" {

// Layout bytes for (type, n_out, n_in, G); -1 if no layout.
int64_t emu_layout_bytes(uint32_t type, int64_t n_out, int64_t n_in, int G) {
    Layout L;
    if (!make_layout(type, n_out, n_in, G, &L)) return -1;
    return L.total_bytes;
}

// Repack GGUF rows into the planar layout (dev must hold emu_layout_bytes).
int emu_repack(uint32_t type, int64_t n_out, int64_t n_in, int G, const uint8_t *rows,
               uint8_t *dev) {
    Layout L;
    uint32_t be, bb;
    if (!make_layout(type, n_out, n_in, G, &L) || !geometry(type, &be, &bb)) return -1;
    memset(dev, 0, (size_t)L.total_bytes);
    const int64_t row_bytes = n_in / be * bb;
    const int64_t recs = type == T_F16 ? n_in / 32 : n_in / be;
    const int64_t rec_bytes = type == T_F16 ? 64 : bb;
    for (int64_t row = 0; row < n_out; row++)
        for (int64_t k = 0; k < recs; k++)
            repack_block(L, dev, rows + row * row_bytes + k * rec_bytes, row, k);
    return 0;
}

// Full emulated matvec: rows (GGUF bytes) x pair-format activation -> y,
// with column slices of about slice_elems elements (< 0: the library's
// default kSliceElems, 0: none).
int emu_gemv_pair(uint32_t type, int64_t n_out, int64_t n_in, int G, int64_t slice_elems,
                  const uint8_t *rows, const uint8_t *xq, float *y) {
    Layout L;
    if (!make_layout(type, n_out, n_in, G, &L)) return -1;
    const int64_t spr = slice_rounds(L, slice_elems < 0 ? kSliceElems : slice_elems);
    std::vector<uint8_t> dev((size_t)L.total_bytes);
    if (emu_repack(type, n_out, n_in, G, rows, dev.data())) return -1;
    const uint32_t pair = pair_of(type);
    const int64_t cb = lds_col(pair, n_in);
    std::vector<uint8_t> lds((size_t)cb, 0);
    stage(pair, n_in, xq, lds.data());
    switch (type) {
        case T_F16:  run<T_F16>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q4_0: run<T_Q4_0>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q5_0: run<T_Q5_0>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q8_0: run<T_Q8_0>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q2_K: run<T_Q2_K>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q3_K: run<T_Q3_K>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q4_K: run<T_Q4_K>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q5_K: run<T_Q5_K>(L, dev.data(), lds.data(), cb, spr, y); break;
        case T_Q6_K: run<T_Q6_K>(L, dev.data(), lds.data(), cb, spr, y); break;
        default: return -1;
    }
    return 0;
}

// Dequantize every row of a repacked matrix through the planar layout (the
// device kernel's indexing): out[row * n_in + i].
int emu_dequant(uint32_t type, int64_t n_out, int64_t n_in, int G, const uint8_t *rows, float *out) {
    Layout L;
    if (!make_layout(type, n_out, n_in, G, &L)) return -1;
    std::vector<uint8_t> dev((size_t)L.total_bytes);
    if (emu_repack(type, n_out, n_in, G, rows, dev.data())) return -1;
    Planes P;
    for (int p = 0; p < 4; p++) P.p[p] = dev.data() + L.plane_off[p];
    for (int64_t row = 0; row < n_out; row++) {
        for (int64_t c = 0; c < L.ncols; c++) {
            const uint32_t cr = (uint32_t)col_rec(L, row, c);
            float *o = out + row * n_in;
            if (is_kquant(type)) {
                KRaw w;
                const uint32_t urec = (cr >> 6) * 512u + (cr & 63u);
                switch (type) {
                    case T_Q2_K: load_kblock<T_Q2_K>(P, urec, cr, w); break;
                    case T_Q3_K: load_kblock<T_Q3_K>(P, urec, cr, w); break;
                    case T_Q4_K: load_kblock<T_Q4_K>(P, urec, cr, w); break;
                    case T_Q5_K: load_kblock<T_Q5_K>(P, urec, cr, w); break;
                    default: load_kblock<T_Q6_K>(P, urec, cr, w); break;
                }
                for (int k = 0; k < 8; k++) {
                    float *u = o + c * 256 + 32 * k;
                    switch (type) {
                        case T_Q2_K: dequant_kunit<T_Q2_K>(w, k, u); break;
                        case T_Q3_K: dequant_kunit<T_Q3_K>(w, k, u); break;
                        case T_Q4_K: dequant_kunit<T_Q4_K>(w, k, u); break;
                        case T_Q5_K: dequant_kunit<T_Q5_K>(w, k, u); break;
                        default: dequant_kunit<T_Q6_K>(w, k, u); break;
                    }
                }
            } else {
                Raw w;
                float *u = o + c * 32;
                switch (type) {
                    case T_Q4_0: load_unit<T_Q4_0>(P, cr, w); dequant_unit<T_Q4_0>(w, u); break;
                    case T_Q5_0: load_unit<T_Q5_0>(P, cr, w); dequant_unit<T_Q5_0>(w, u); break;
                    case T_Q8_0: load_unit<T_Q8_0>(P, cr, w); dequant_unit<T_Q8_0>(w, u); break;
                    default: load_unit<T_F16>(P, cr, w); dequant_unit<T_F16>(w, u); break;
                }
            }
        }
    }
    return 0;
}

}  // extern "C"
