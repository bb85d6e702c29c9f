// Device-side weight layout for the quantized matvec path (gfx950).
//
// GGUF blocks (reference include/siphon/quant.h:31-100) are packed for a
// scalar CPU reader: 18/22/34/84/110/144/176/210-byte records that are not
// 16-byte aligned and interleave scales with quants. On the device every
// weight matrix is stored instead as a set of PLANES, each holding one kind
// of field, laid out so that one wavefront load instruction reads one
// contiguous span (64 lanes x plane bytes):
//
//   unit   = 32 consecutive elements of a row (one 32-block for Q4_0/Q5_0/
//            Q8_0/F16, one eighth of a 256-element super-block for K-quants)
//   column = what one lane handles per round: a whole super-block (K-quants,
//            8 units, so its scales are loaded and unpacked once) or a unit
//   (tile geometry and record order: see Layout below)
//
// Inside a unit the quantized values are re-packed to one canonical order so
// that every format decodes to 8 dwords q[t], byte k of q[t] = element 4t+k,
// ready for v_dot4 against the activation bytes in natural order:
//   nib16 (16 B): byte k = v[k] | v[16 + k] << 4
//   bit4  ( 4 B): bit 8k + t of the u32 = 1-bit value of element 4t + k
//   two8  ( 8 B): u32 h[e / 16]; bits 8k + 2t .. +1 of h[i] = 2-bit value of
//                 element 16i + 4t + k
// The repacking is a bijection on the bits: device bytes equal GGUF bytes
// (plus zero-filled tile padding).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define SIHD __host__ __device__
#else
#define SIHD
#endif

namespace sihip {

enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q5_0 = 6, T_Q8_0 = 8,
    T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_Q8_K = 15,
};

// GGUF geometry (reference quant.h:92-100).
SIHD inline bool geometry(uint32_t t, uint32_t *be, uint32_t *bb) {
    switch (t) {
        case T_F32:  *be = 1;   *bb = 4;   return true;
        case T_F16:  *be = 1;   *bb = 2;   return true;
        case T_Q4_0: *be = 32;  *bb = 18;  return true;
        case T_Q5_0: *be = 32;  *bb = 22;  return true;
        case T_Q8_0: *be = 32;  *bb = 34;  return true;
        case T_Q2_K: *be = 256; *bb = 84;  return true;
        case T_Q3_K: *be = 256; *bb = 110; return true;
        case T_Q4_K: *be = 256; *bb = 144; return true;
        case T_Q5_K: *be = 256; *bb = 176; return true;
        case T_Q6_K: *be = 256; *bb = 210; return true;
        case T_Q8_K: *be = 256; *bb = 292; return true;
        default: return false;
    }
}

// Activation pair format (reference kernels.c:946-960).
SIHD constexpr inline uint32_t pair_of(uint32_t t) {
    switch (t) {
        case T_F32: return T_F32;
        case T_F16: return T_F16;
        case T_Q4_0: case T_Q5_0: case T_Q8_0: return T_Q8_0;
        default: return T_Q8_K;
    }
}

SIHD constexpr inline bool is_kquant(uint32_t t) {
    return t == T_Q2_K || t == T_Q3_K || t == T_Q4_K || t == T_Q5_K || t == T_Q6_K;
}

// Plane table: bytes per record and whether the record is per unit (0) or
// per super-block (1). Order is the order of planes in device memory.
struct PlaneSpec {
    int n;
    int bytes[4];
    int per_block[4];
};

SIHD inline PlaneSpec planes_of(uint32_t t) {
    switch (t) {
        case T_F16:  return {1, {64, 0, 0, 0}, {0, 0, 0, 0}};
        case T_Q4_0: return {2, {16, 2, 0, 0}, {0, 0, 0, 0}};
        case T_Q5_0: return {3, {16, 4, 2, 0}, {0, 0, 0, 0}};
        case T_Q8_0: return {2, {32, 2, 0, 0}, {0, 0, 0, 0}};
        case T_Q2_K: return {3, {8, 16, 4, 0}, {0, 1, 1, 0}};
        case T_Q3_K: return {4, {8, 4, 12, 2}, {0, 0, 1, 1}};
        case T_Q4_K: return {2, {16, 16, 0, 0}, {0, 1, 0, 0}};
        case T_Q5_K: return {3, {16, 4, 16, 0}, {0, 0, 1, 0}};
        case T_Q6_K: return {4, {16, 8, 16, 2}, {0, 0, 1, 1}};
        default:     return {0, {0, 0, 0, 0}, {0, 0, 0, 0}};
    }
}

// Geometry of one uploaded matrix in the planar layout.
//
// A row is a sequence of COLUMNS: super-blocks of 256 elements for the
// K-quants, 32-element units for Q4_0/Q5_0/Q8_0/F16. A wave tile covers R
// rows x G columns (R * G = 64, lane = r * G + g); round s of the tile gives
// lane (r, g) column c = s * G + g of row tile * R + r. When G does not
// divide the column count, the last round has padding slots past the row:
// they are allocated (zero-filled) but the matvec kernel does not read them
// (it re-reads a real column of the row and discards the result). Rows past
// n_out in the last tile are zero-filled and read.
//   column-level plane record = (tile * S + s) * 64 + lane
//   unit-level plane record (K-quants, unit k = 0..7 of the super-block)
//                            = ((tile * S + s) * 8 + k) * 64 + lane
// so every load instruction of a wave reads 64 consecutive records.
struct Layout {
    uint32_t type;
    int64_t n_out, n_in;
    int64_t nunits;   // n_in / 32
    int64_t ncols;    // columns per row: n_in / 256 (K-quants) or n_in / 32
    int G, R;         // columns and rows per wave tile (G * R = 64)
    int logG;
    int64_t S;        // rounds per tile = ceil(ncols / G)
    int64_t ntiles;   // ceil(n_out / R)
    int nplanes;
    int64_t plane_off[4];
    int plane_bytes[4];
    int plane_blk[4];  // 1: one record per super-block (K-quants)
    int64_t total_bytes;
};

SIHD inline int64_t plane_records(const Layout &L, int p) {
    const bool unit_level = is_kquant(L.type) && !L.plane_blk[p];
    return L.ntiles * L.S * 64 * (unit_level ? 8 : 1);
}

inline bool make_layout(uint32_t type, int64_t n_out, int64_t n_in, int G, Layout *L) {
    uint32_t be, bb;
    if (!geometry(type, &be, &bb) || type == T_Q8_K || type == T_F32) return false;  // F32: no planes
    if (n_in <= 0 || n_out <= 0 || n_in % 32 != 0 || n_in % be != 0) return false;
    if (G < 1 || G > 64 || (G & (G - 1))) return false;
    L->type = type;
    L->n_out = n_out;
    L->n_in = n_in;
    L->nunits = n_in / 32;
    L->ncols = is_kquant(type) ? n_in / 256 : n_in / 32;
    L->G = G;
    L->R = 64 / G;
    L->logG = 0;
    while ((1 << L->logG) < G) L->logG++;
    L->S = (L->ncols + G - 1) / G;
    L->ntiles = (n_out + L->R - 1) / L->R;
    const PlaneSpec ps = planes_of(type);
    L->nplanes = ps.n;
    int64_t off = 0;
    for (int p = 0; p < 4; p++) {
        L->plane_bytes[p] = ps.bytes[p];
        L->plane_blk[p] = ps.per_block[p];
        L->plane_off[p] = off;
        if (p < ps.n) {
            const int64_t pb = plane_records(*L, p) * ps.bytes[p];
            if (pb >= ((int64_t)1 << 32)) return false;  // kernels use 32-bit offsets
            off += pb;
            off = (off + 255) & ~(int64_t)255;
        }
    }
    L->total_bytes = off;
    return true;
}

// Column slices of long rows. A matvec workgroup that computes whole rows
// first converts the whole activation row into LDS; for long rows that
// prologue outweighs the workgroup's share of the streaming. Rows of at
// least 2 * kSliceElems elements are cut into slices of about kSliceElems
// activation elements (whole rounds of the tile), each computed by its own
// workgroups; the partial sums of a row are added in slice order.
// slice_rounds() gives the rounds per slice, L.S (one slice) for shorter
// rows or elems <= 0.
constexpr int64_t kSliceElems = 4096;

// Rows shorter than 2 * kSliceElems are never sliced, whatever the slice
// length (a shorter slice only cuts the long rows finer).
SIHD inline bool sliced_rows(int64_t n_in, int64_t elems) {
    return elems > 0 && n_in >= 2 * elems && n_in >= 2 * kSliceElems;
}

SIHD inline int64_t slice_rounds(const Layout &L, int64_t elems) {
    const int64_t col_elems = is_kquant(L.type) ? 256 : 32;
    if (!sliced_rows(L.n_in, elems)) return L.S;
    int64_t r = elems / (L.G * col_elems);
    if (r < 1) r = 1;
    return r < L.S ? r : L.S;
}

// Record index of column c of row `row` (column-level planes).
SIHD inline int64_t col_rec(const Layout &L, int64_t row, int64_t c) {
    const int64_t tile = row / L.R, r = row % L.R;
    const int64_t s = c >> L.logG, g = c & (L.G - 1);
    return (tile * L.S + s) * 64 + r * L.G + g;
}

// Byte offset of unit u of row `row` in unit plane p.
SIHD inline int64_t unit_off(const Layout &L, int p, int64_t row, int64_t u) {
    if (is_kquant(L.type)) {
        const int64_t cr = col_rec(L, row, u >> 3);  // (tile*S + s)*64 + lane
        const int64_t rec = ((cr >> 6) * 8 + (u & 7)) * 64 + (cr & 63);
        return L.plane_off[p] + rec * L.plane_bytes[p];
    }
    return L.plane_off[p] + col_rec(L, row, u) * L.plane_bytes[p];
}

// Byte offset of the super-block containing unit u in block plane p.
SIHD inline int64_t block_off(const Layout &L, int p, int64_t row, int64_t u) {
    return L.plane_off[p] + col_rec(L, row, u >> 3) * L.plane_bytes[p];
}

// ---- canonical packers (one unit of 32 values) ---------------------------

SIHD inline void pack_nib16(const uint8_t v[32], uint8_t out[16]) {
    for (int k = 0; k < 16; k++) out[k] = (uint8_t)((v[k] & 15) | ((v[16 + k] & 15) << 4));
}

SIHD inline uint32_t pack_bit4(const uint8_t v[32]) {
    uint32_t h = 0;
    for (int t = 0; t < 8; t++)
        for (int k = 0; k < 4; k++) h |= (uint32_t)(v[4 * t + k] & 1) << (8 * k + t);
    return h;
}

SIHD inline void pack_two8(const uint8_t v[32], uint32_t h[2]) {
    h[0] = h[1] = 0;
    for (int i = 0; i < 2; i++)
        for (int t = 0; t < 4; t++)
            for (int k = 0; k < 4; k++)
                h[i] |= (uint32_t)(v[16 * i + 4 * t + k] & 3) << (8 * k + 2 * t);
}

SIHD inline void put32(uint8_t *p, uint32_t v) {
    p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24);
}

// ---- repack one GGUF block into the planes --------------------------------
// blk points at the GGUF bytes of block `kb` of row `row` (kb counts blocks
// of be elements). Values per element follow the reference dequantizers
// (reference kernels.c:599-817); only their bit placement changes.

SIHD inline void repack_block(const Layout &L, uint8_t *dev, const uint8_t *blk,
                              int64_t row, int64_t kb) {
    uint8_t v[32];
    switch (L.type) {
        case T_F16: {  // kb counts 32-element units here (see caller)
            uint8_t *o = dev + unit_off(L, 0, row, kb);
            for (int i = 0; i < 64; i++) o[i] = blk[i];
            return;
        }
        case T_Q4_0: {
            uint8_t *o = dev + unit_off(L, 0, row, kb);
            for (int k = 0; k < 16; k++) o[k] = blk[2 + k];  // already nib16
            uint8_t *d = dev + unit_off(L, 1, row, kb);
            d[0] = blk[0]; d[1] = blk[1];
            return;
        }
        case T_Q5_0: {
            uint8_t *o = dev + unit_off(L, 0, row, kb);
            for (int k = 0; k < 16; k++) o[k] = blk[6 + k];
            const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) |
                                ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
            for (int e = 0; e < 32; e++) v[e] = (uint8_t)((qh >> e) & 1);
            put32(dev + unit_off(L, 1, row, kb), pack_bit4(v));
            uint8_t *d = dev + unit_off(L, 2, row, kb);
            d[0] = blk[0]; d[1] = blk[1];
            return;
        }
        case T_Q8_0: {
            uint8_t *o = dev + unit_off(L, 0, row, kb);
            for (int k = 0; k < 32; k++) o[k] = blk[2 + k];
            uint8_t *d = dev + unit_off(L, 1, row, kb);
            d[0] = blk[0]; d[1] = blk[1];
            return;
        }
        default: break;
    }
    // K-quants: 8 units per super-block
    const int64_t u0 = kb * 8;
    switch (L.type) {
        case T_Q2_K: {
            const uint8_t *sc = blk, *qs = blk + 16;
            for (int j = 0; j < 8; j++) {
                const int h = j >> 2, s = j & 3;
                for (int l = 0; l < 32; l++) v[l] = (uint8_t)((qs[32 * h + l] >> (2 * s)) & 3);
                uint32_t hh[2];
                pack_two8(v, hh);
                uint8_t *o = dev + unit_off(L, 0, row, u0 + j);
                put32(o, hh[0]); put32(o + 4, hh[1]);
            }
            uint8_t *o1 = dev + block_off(L, 1, row, u0);
            for (int k = 0; k < 16; k++) o1[k] = sc[k];
            uint8_t *o2 = dev + block_off(L, 2, row, u0);
            for (int k = 0; k < 4; k++) o2[k] = blk[80 + k];  // d, dmin
            return;
        }
        case T_Q3_K: {
            const uint8_t *hm = blk, *qs = blk + 32;
            for (int j = 0; j < 8; j++) {
                const int h = j >> 2, s = j & 3;
                uint8_t hb[32];
                for (int l = 0; l < 32; l++) {
                    v[l] = (uint8_t)((qs[32 * h + l] >> (2 * s)) & 3);
                    hb[l] = (uint8_t)((hm[l] >> (4 * h + s)) & 1);
                }
                uint32_t hh[2];
                pack_two8(v, hh);
                uint8_t *o = dev + unit_off(L, 0, row, u0 + j);
                put32(o, hh[0]); put32(o + 4, hh[1]);
                put32(dev + unit_off(L, 1, row, u0 + j), pack_bit4(hb));
            }
            uint8_t *o2 = dev + block_off(L, 2, row, u0);
            for (int k = 0; k < 12; k++) o2[k] = blk[96 + k];
            uint8_t *o3 = dev + block_off(L, 3, row, u0);
            o3[0] = blk[108]; o3[1] = blk[109];
            return;
        }
        case T_Q4_K:
        case T_Q5_K: {
            const bool five = L.type == T_Q5_K;
            const uint8_t *qh = blk + 16, *qs = blk + (five ? 48 : 16);
            for (int j = 0; j < 8; j++) {
                const int c = j >> 1, hi = j & 1;
                for (int l = 0; l < 32; l++)
                    v[l] = (uint8_t)(hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15));
                pack_nib16(v, dev + unit_off(L, 0, row, u0 + j));
                if (five) {
                    for (int l = 0; l < 32; l++) v[l] = (uint8_t)((qh[l] >> j) & 1);
                    put32(dev + unit_off(L, 1, row, u0 + j), pack_bit4(v));
                }
            }
            uint8_t *om = dev + block_off(L, five ? 2 : 1, row, u0);
            for (int k = 0; k < 16; k++) om[k] = blk[k];  // d, dmin, scales[12]
            return;
        }
        case T_Q6_K: {
            const uint8_t *ql = blk, *qh = blk + 128;
            for (int j = 0; j < 8; j++) {
                const int h = j >> 2, t = j & 3;
                uint8_t hi2[32];
                for (int l = 0; l < 32; l++) {
                    const uint8_t byte = ql[64 * h + l + 32 * (t & 1)];
                    v[l] = (uint8_t)(t < 2 ? (byte & 15) : (byte >> 4));
                    hi2[l] = (uint8_t)((qh[32 * h + l] >> (2 * t)) & 3);
                }
                pack_nib16(v, dev + unit_off(L, 0, row, u0 + j));
                uint32_t hh[2];
                pack_two8(hi2, hh);
                uint8_t *o = dev + unit_off(L, 1, row, u0 + j);
                put32(o, hh[0]); put32(o + 4, hh[1]);
            }
            uint8_t *o2 = dev + block_off(L, 2, row, u0);
            for (int k = 0; k < 16; k++) o2[k] = blk[192 + k];
            uint8_t *o3 = dev + block_off(L, 3, row, u0);
            o3[0] = blk[208]; o3[1] = blk[209];
            return;
        }
        default: return;
    }
}

}  // namespace sihip
