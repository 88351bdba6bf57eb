// qh_mmv16.hip -- staged matrix-core GEMV for the 256-weight superblock formats
// (Q4_K, Q5_K, Q6_K) on v_mfma_i32_16x16x64_i8.
//
// Workgroup = ROWS (<= 16) output rows x W wavefronts that split K.  A wavefront
// works on chunks of GPW superblock columns ("groups" of 256 weights):
//   1. it loads the chunk's x first (one float4 per lane per group), then the
//      chunk's weight bytes with fully coalesced 16-byte buffer loads: lane q of a
//      group's load covers slice q % CH of row q / CH (ROWS x CH x 16 bytes);
//   2. x is turned into three balanced int8 digit planes in LDS (the exponent is
//      per wavefront and chunk, so the int32 MFMA sums are exact);
//   3. per group, the wavefront writes its slices into a private LDS tile (one
//      QH_RS-byte line per row, 16-byte aligned whatever the block alignment in
//      memory) and reads them back transposed: lane (n = lane % 16, kg = lane / 16)
//      owns two 16-byte chunks of row n's quants and turns their low and high
//      nibbles into the B operands (column n) of the group's four MFMAs.  Every
//      B operand is 16 weights that share one scale ("piece" = 16 consecutive x
//      positions).  The A operand of MFMA s holds, in row 4 kg + m only, digit m of
//      the x piece that lane kg's B operand multiplies, so result row 4 kg + m,
//      column n (returned in lane 16 kg + n, register m) is the digit-m dot of that
//      lane's own piece: each lane applies its piece's integer scale, no shuffles.
//   4. sums over lanes and wavefronts finish through DPP/LDS.
//
// Reference counterpart: the warp-per-row cuda_gemv kernels of
// src/cuda_kernels.cu:1046-1077 (one f32 FMA per weight).
#include <climits>
#include <type_traits>

#include "qh_formats.h"
#include "qh_internal.h"

typedef int32_t qh_i32x4 __attribute__((ext_vector_type(4)));

// x of one group in LDS: digit plane m of piece q at 256m + 16q, the f32 sum of
// piece q at 768 + 4q, and 16 zero bytes (the A operand of lanes that carry no
// digits) at 832.
#define QH_XG 1024
#define QH_XG_SUM 768
#define QH_XG_ZERO 832
#define QH_RS 240   // LDS line per row: 15 x 16 bytes, conflict-free b128 reads over 16 rows
#define QH_MAXT 64  // row tiles per workgroup (their results wait in LDS until the end)
#define QH_RING 4   // finished tiles per workgroup barrier (launches with few tiles)

QH_DEV uint32_t qh_lo4(uint32_t q) { return q & 0x0F0F0F0Fu; }
// Formats whose blocks sit at 2-byte alignment set HALF: a 16-byte load at an
// address that is not a multiple of 4 costs the address units far more than
// one at a multiple of 4 (measured on MI355X: the Q6_K head 86 against 73 us),
// so their slices are loaded from the dword at or below the slice and shifted
// into place when staged, the two bytes past them taken from the next lane's
// load (the next slice of the row).  The last slice starts at a multiple of 4
// from the block (LAST), so its two missing bytes lie past the block.
template <class F, class = void>
struct QhHalf : std::false_type {};
template <class F>
struct QhHalf<F, std::void_t<decltype(F::HALF)>> : std::bool_constant<F::HALF> {};
QH_DEV uint32_t qh_hi4(uint32_t q) { return (q >> 4) & 0x0F0F0F0Fu; }

// ---------------------------------------------------------------- formats
// Each format gives: BYTES (per superblock), CH (16-byte slices loaded per row and
// superblock; slice c starts at block byte 16c, the last at LAST <= BYTES - 14),
// ROWS, a header decoded once per group (hdr), the four B operands of lane kg
// (bops), and per MFMA s: the x piece of lane kg (piece), its integer scale (scl)
// and the integer weight of the piece's f32 x-sum (mn).  Group result:
//   y += d * 2^-s * sum(scl * digit dots) - dm * sum(mn * xsum).

// Q4_K: d, dmin, scales[12], qs[128] (src/dequant.rs:1471-1519).  Weight = d*sc*q - dmin*m.
// Lane kg owns qs chunks c = kg (MFMAs 0, 1 = low, high nibbles) and c = kg + 4
// (MFMAs 2, 3).  qs chunk c holds sub-blocks 2(c/2) (low) and 2(c/2)+1 (high),
// positions 16(c%2) .. +15.
struct M16Q4K {
    static constexpr int BYTES = 144, CH = 9, ROWS = 14, LAST = 128, RS = QH_RS;
    static constexpr bool FLOAT_D = false, MINS = true;
    static constexpr int GRID = 0;
    struct H { uint32_t sc0, sc1, mn0, mn1; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r, int) {
        const qh_u32x4 h = *reinterpret_cast<const qh_u32x4*>(r);
        H o;
        o.sc0 = h.y & 0x3F3F3F3Fu;
        o.mn0 = h.z & 0x3F3F3F3Fu;
        o.sc1 = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
        o.mn1 = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
        o.d = qh_f16_lo(h.x);
        o.dm = qh_f16_hi(h.x);
        return o;
    }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char*) {
        const qh_u32x4 q0 = *reinterpret_cast<const qh_u32x4*>(r + 16 + 16 * kg);
        const qh_u32x4 q1 = *reinterpret_cast<const qh_u32x4*>(r + 80 + 16 * kg);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            B[0][i] = (int)qh_lo4(q0[i]);
            B[1][i] = (int)qh_hi4(q0[i]);
            B[2][i] = (int)qh_lo4(q1[i]);
            B[3][i] = (int)qh_hi4(q1[i]);
        }
    }
    // sub-block j = 2(kg/2) + 4(S/2) + S%2, piece = 2j + kg%2.
    template <int S>
    static QH_DEV int piece(int kg) { return 4 * (kg >> 1) + 8 * (S >> 1) + 2 * (S & 1) + (kg & 1); }
    template <int S>
    static QH_DEV int scl(const H& h, int kg) {
        return (int)(((S < 2 ? h.sc0 : h.sc1) >> (16 * (kg >> 1) + 8 * (S & 1))) & 0xFFu);
    }
    template <int S>
    static QH_DEV int mn(const H& h, int kg) {
        return (int)(((S < 2 ? h.mn0 : h.mn1) >> (16 * (kg >> 1) + 8 * (S & 1))) & 0xFFu);
    }
};

// Q5_K: d, dmin, scales[12], qh[32], qs[128] (src/dequant.rs:1146-1182).
// Weight of sub-block j, position l: d*sc*(nibble + 16*bit_j(qh[l])) - dmin*m.
// Chunks as Q4_K (qs at byte 48); both of lane kg's chunks use qh[16(kg%2) ..].
struct M16Q5K {
    static constexpr int BYTES = 176, CH = 11, ROWS = 11, LAST = 160, RS = QH_RS;
    static constexpr bool FLOAT_D = false, MINS = true;
    static constexpr int GRID = 0;
    using H = M16Q4K::H;
    static QH_DEV H hdr(const unsigned char* r, int kg) { return M16Q4K::hdr(r, kg); }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char*) {
        const qh_u32x4 q0 = *reinterpret_cast<const qh_u32x4*>(r + 48 + 16 * kg);
        const qh_u32x4 q1 = *reinterpret_cast<const qh_u32x4*>(r + 112 + 16 * kg);
        const qh_u32x4 u = *reinterpret_cast<const qh_u32x4*>(r + 16 + 16 * (kg & 1));
        const uint32_t j = 2u * (uint32_t)(kg >> 1);  // sub-block of chunk kg's low nibbles
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = u[i] >> j;
            B[0][i] = (int)(qh_lo4(q0[i]) | ((v & 0x01010101u) << 4));
            B[1][i] = (int)(qh_hi4(q0[i]) | ((v & 0x02020202u) << 3));
            B[2][i] = (int)(qh_lo4(q1[i]) | ((v & 0x10101010u)));
            B[3][i] = (int)(qh_hi4(q1[i]) | ((v & 0x20202020u) >> 1));
        }
    }
    template <int S>
    static QH_DEV int piece(int kg) { return M16Q4K::piece<S>(kg); }
    template <int S>
    static QH_DEV int scl(const H& h, int kg) { return M16Q4K::scl<S>(h, kg); }
    template <int S>
    static QH_DEV int mn(const H& h, int kg) { return M16Q4K::mn<S>(h, kg); }
};

// Q6_K: ql[128], qh[64], scales[16] (int8), d (src/dequant.rs:1583-1620).
// Half n, ql[64n + l] low nibble = position 128n + l, high = 128n + 64 + l;
// qh[32n + l'] bits 2i..2i+1 = bits 4-5 of position 128n + 32i + l'.
// Lane kg owns ql chunks kg (half 0) and kg + 4 (half 1): MFMA s = (half s/2,
// nibble s%2) covers piece 8(s/2) + 4(s%2) + kg, whose scale is byte kg of
// scales word s.  Weight = d*sc*(q - 32): the -32 goes through the x sums.
struct M16Q6K {
    static constexpr int BYTES = 210, CH = 14, ROWS = 16;
    // The 14th slice is block bytes 196-211 (a multiple of 4 from the block, as
    // HALF needs; the last two bytes are past the block and unused): the LDS
    // line holds bytes 0-207 at 0-207 and d at 220.
    static constexpr int LAST = 196, RS = QH_RS;
    static constexpr bool FLOAT_D = false, MINS = true, HALF = true;
    static constexpr int GRID = 0;
    struct H { qh_u32x4 s; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r, int) {
        H o;
        o.s = *reinterpret_cast<const qh_u32x4*>(r + 192);
        o.d = qh_h2f(*reinterpret_cast<const uint16_t*>(r + 208 + (BYTES - 2 - LAST)));
        o.dm = 32.0f * o.d;
        return o;
    }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char*) {
        const qh_u32x4 l0 = *reinterpret_cast<const qh_u32x4*>(r + 16 * kg);
        const qh_u32x4 l1 = *reinterpret_cast<const qh_u32x4*>(r + 64 + 16 * kg);
        const qh_u32x4 u0 = *reinterpret_cast<const qh_u32x4*>(r + 128 + 16 * (kg & 1));
        const qh_u32x4 u1 = *reinterpret_cast<const qh_u32x4*>(r + 160 + 16 * (kg & 1));
        const uint32_t sh = 2u * (uint32_t)(kg >> 1);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v0 = u0[i] >> sh, v1 = u1[i] >> sh;
            B[0][i] = (int)(qh_lo4(l0[i]) | ((v0 & 0x03030303u) << 4));
            B[1][i] = (int)(qh_hi4(l0[i]) | (v0 & 0x30303030u));
            B[2][i] = (int)(qh_lo4(l1[i]) | ((v1 & 0x03030303u) << 4));
            B[3][i] = (int)(qh_hi4(l1[i]) | (v1 & 0x30303030u));
        }
    }
    template <int S>
    static QH_DEV int piece(int kg) { return 8 * (S >> 1) + 4 * (S & 1) + kg; }
    template <int S>
    static QH_DEV int scl(const H& h, int kg) { return ((int)(h.s[S] >> (8 * kg)) << 24) >> 24; }
    template <int S>
    static QH_DEV int mn(const H& h, int kg) { return scl<S>(h, kg); }
};

// Q6_K for K past one chunk (in_dim > 4096): plain 2-byte aligned loads, the
// last slice from block bytes 194-209 (d at line 222).  With many chunks per
// wavefront the shifts of HALF cost more than they save (4096x14336: 12.2 us
// plain, 13.0 with HALF).
struct M16Q6KW : M16Q6K {
    static constexpr int LAST = 194;
    static constexpr bool HALF = false;
    static QH_DEV H hdr(const unsigned char* r, int) {
        H o;
        o.s = *reinterpret_cast<const qh_u32x4*>(r + 192);
        o.d = qh_h2f(*reinterpret_cast<const uint16_t*>(r + 208 + (BYTES - 2 - LAST)));
        o.dm = 32.0f * o.d;
        return o;
    }
};

// Q8_0: blocks of [d f16][32 x int8] (src/dequant.rs:1450-1463); a group is 8
// blocks (272 bytes, so groups stay 16-byte aligned in a row).  Piece p (16
// weights) is half p % 2 of block p / 2: its quants are the B operand as they
// are (int8), read with an unaligned ds_read_b128 at block byte 2 + 16 (p % 2);
// each piece has its own f32 scale d (FLOAT_D), no mins.  Line stride 272 B
// puts the 16 rows of a column 4 banks apart.
struct M16Q80 {
    static constexpr int BYTES = 272, CH = 17, ROWS = 15, LAST = 256, RS = 272;
    static constexpr bool FLOAT_D = true, MINS = false;
    static constexpr int GRID = 0;
    struct H { float d[4]; float dm; };
    template <int S>
    static QH_DEV int piece(int kg) { return 4 * S + kg; }
    static QH_DEV H hdr(const unsigned char* r, int kg) {
        H o;
#pragma unroll
        for (int s = 0; s < 4; s++) o.d[s] = qh_h2f(*reinterpret_cast<const uint16_t*>(r + 34 * ((4 * s + kg) >> 1)));
        o.dm = 0.f;
        return o;
    }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char*) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int p = 4 * s + kg;
            __builtin_memcpy(&B[s], r + 34 * (p >> 1) + 2 + 16 * (p & 1), 16);
        }
    }
    template <int S>
    static QH_DEV int scl(const H&, int) { return 1; }
    template <int S>
    static QH_DEV int mn(const H&, int) { return 0; }
    template <int S>
    static QH_DEV float dsc(const H& h) { return h.d[S]; }
};

// IQ3_S / IQ2_XXS: signed codebook bytes as the B operand (qh_iq3s_piece /
// qh_iq2xxs_piece), the codebook in the workgroup's LDS (GRID 1 / 2).  Lane kg,
// MFMA s: half kg % 2 of sub-block 2s + kg / 2, i.e. piece 4s + kg; its scale is
// the sub-block's odd integer, no mins.
struct M16IQ3S {
    static constexpr int BYTES = 110, CH = 7, ROWS = 16, LAST = 94, RS = QH_RS;
    static constexpr bool FLOAT_D = false, MINS = false;
    static constexpr int GRID = 1;
    struct H { int sc[4]; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r, int kg) {
        H o;
        // scales[0..3] sit at LDS 108..111 (block bytes 106..109)
        const uint32_t s4 = *reinterpret_cast<const uint32_t*>(r + qh_iq3s_at(106));
        const int nib = 4 * ((kg >> 1) & 1);
#pragma unroll
        for (int s = 0; s < 4; s++) o.sc[s] = 1 + 2 * (int)((s4 >> (8 * s + nib)) & 0xFu);
        o.d = qh_h2f(qh_rd16(r, 0));
        o.dm = 0.f;
        return o;
    }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char* grid) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            uint32_t v[4];
            int sc;
            qh_iq3s_piece(r, 2 * s + (kg >> 1), kg & 1, reinterpret_cast<const uint32_t*>(grid), v, sc);
#pragma unroll
            for (int m = 0; m < 4; m++) B[s][m] = (int)v[m];
        }
    }
    template <int S>
    static QH_DEV int piece(int kg) { return 4 * S + kg; }
    template <int S>
    static QH_DEV int scl(const H& h, int) { return h.sc[S]; }
    template <int S>
    static QH_DEV int mn(const H&, int) { return 0; }
};

struct M16IQ2XXS {
    static constexpr int BYTES = 66, CH = 5, ROWS = 16, LAST = 50, RS = QH_RS;
    static constexpr bool FLOAT_D = false, MINS = false;
    static constexpr int GRID = 2;
    struct H { int sc[4]; float d, dm; };
    static QH_DEV H hdr(const unsigned char* r, int kg) {
        H o;
#pragma unroll
        for (int s = 0; s < 4; s++) o.sc[s] = 2 * (int)(r[qh_iq2xxs_at(9 + 8 * (2 * s + (kg >> 1)))] >> 4) + 1;
        o.d = 0.125f * qh_h2f(qh_rd16(r, 0));
        o.dm = 0.f;
        return o;
    }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char* grid) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            uint32_t v[4];
            int sc;
            qh_iq2xxs_piece(r, 2 * s + (kg >> 1), kg & 1, reinterpret_cast<const uint64_t*>(grid), v, sc);
#pragma unroll
            for (int m = 0; m < 4; m++) B[s][m] = (int)v[m];
        }
    }
    template <int S>
    static QH_DEV int piece(int kg) { return 4 * S + kg; }
    template <int S>
    static QH_DEV int scl(const H& h, int) { return h.sc[S]; }
    template <int S>
    static QH_DEV int mn(const H&, int) { return 0; }
};

// The 32-element block formats (src/dequant.rs:1381-1443 Q5_0/Q5_1, :1527-1574
// IQ4_NL; Q4_0/Q4_1 by the public GGUF layout): a group is 8 blocks (16-byte
// aligned in a row when in_dim % 256 == 0).  Piece p = half p % 2 of block
// p / 2, 16 quants as the int8 B operand with the block's own f32 scale d
// (FLOAT_D); the offset of Q4_0 / Q5_0 (-8 / -16) and IQ4_NL's codebook go into
// the bytes, the minimum m of Q4_1 / Q5_1 through the piece's x sum.
// Dispatched for Q4_1 and Q5_1 only: their quants sit 4- and 8-byte aligned in
// the staged line; the 18- and 22-byte blocks of Q4_0, IQ4_NL and Q5_0 leave
// them 2-byte aligned, and those measured no faster (Q5_0: 23.4 against 15.1 us
// at 14336x4096) than the VALU kernel, which keeps them.
template <int KIND>  // 0 Q4_0, 1 Q4_1, 2 Q5_0, 3 Q5_1, 4 IQ4_NL
struct M16Blk {
    static constexpr int BB = (KIND == 0 || KIND == 4) ? 18 : (KIND == 1 ? 20 : (KIND == 2 ? 22 : 24));
    static constexpr int QS = (KIND == 0 || KIND == 4) ? 2 : (KIND == 1 ? 4 : (KIND == 2 ? 6 : 8));  // quants
    static constexpr int BYTES = 8 * BB, CH = BYTES / 16, ROWS = 128 / CH, LAST = BYTES - 16, RS = QH_RS;
    static constexpr bool FLOAT_D = true, MINS = KIND == 1 || KIND == 3;
    static constexpr int GRID = 0;
    struct H { float d[4], m[4]; float dm; };
    template <int S>
    static QH_DEV int piece(int kg) { return 4 * S + kg; }
    static QH_DEV H hdr(const unsigned char* r, int kg) {
        H o;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int blk = (4 * s + kg) >> 1;
            o.d[s] = qh_h2f(*reinterpret_cast<const uint16_t*>(r + BB * blk));
            o.m[s] = MINS ? qh_h2f(*reinterpret_cast<const uint16_t*>(r + BB * blk + 2)) : 0.f;
        }
        o.dm = 0.f;
        return o;
    }
    static QH_DEV void bops(const unsigned char* r, int kg, const H&, qh_i32x4* B, const unsigned char*) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int p = 4 * s + kg, blk = p >> 1, half = p & 1;
            uint32_t w[4];
            __builtin_memcpy(w, r + BB * blk + QS, 16);
            uint32_t hb = 0;
            if constexpr (KIND == 2 || KIND == 3) {
                uint32_t qh;
                __builtin_memcpy(&qh, r + BB * blk + QS - 4, 4);
                hb = half ? qh >> 16 : qh & 0xFFFFu;  // bit j: weight j of the piece
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t q = half ? (w[i] >> 4) & 0x0F0F0F0Fu : w[i] & 0x0F0F0F0Fu;
                if constexpr (KIND == 2 || KIND == 3) q |= qh_spread4((hb >> (4 * i)) & 0xFu) << 4;
                if constexpr (KIND == 0) q = (q + 0x78787878u) ^ 0x80808080u;  // q - 8 as int8 (no carries)
                if constexpr (KIND == 2) q = (q + 0x70707070u) ^ 0x80808080u;  // q - 16
                if constexpr (KIND == 4) q = qh_iq4nl_lut(q) ^ 0x80808080u;    // T[q] (T + 128 flipped)
                B[s][i] = (int)q;
            }
        }
    }
    template <int S>
    static QH_DEV int scl(const H&, int) { return 1; }
    template <int S>
    static QH_DEV int mn(const H&, int) { return 0; }
    template <int S>
    static QH_DEV float dsc(const H& h) { return h.d[S]; }
    template <int S>
    static QH_DEV float mnf(const H& h) { return -h.m[S]; }  // enters as -(-m) * sum(x)
};

// 16-row tiles of the same formats (3 loads per lane and group instead of 2):
// chosen when they spread the tiles more evenly over the CUs (4096 rows = 256
// tiles = one per CU).
struct M16Q4K16 : M16Q4K { static constexpr int ROWS = 16; };
struct M16Q5K16 : M16Q5K { static constexpr int ROWS = 16; };
struct M16Q8016 : M16Q80 { static constexpr int ROWS = 16; };

// ---------------------------------------------------------------- kernel

QH_DEV float qh_dpp_max(float m) {
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0xB1, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x4E, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x141, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x140, 0xF, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x142, 0xA, 0xF, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(m), 0x143, 0xC, 0xF, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 63));
}

// Persistent kernel: workgroup b handles row tiles b, b + gridDim.x, ... (ROWS
// rows each).  A wavefront's work items are (tile, K chunk) pairs; the weight
// loads of the next item are issued before the current one is computed, so every
// wavefront keeps one item of loads in flight for the whole kernel.  When K fits
// one chunk (X1: W * GPW >= in_dim / 256), x is digitised once per workgroup.
// Up to QH_MULTI weight matrices sharing x, type and in_dim, computed in one
// launch: their row tiles form one index space (matrix m owns tiles tstart[m] ..
// tstart[m+1]-1); a single GEMV is the one-matrix case.
#define QH_MULTI 4
struct QhMats {
    const uint8_t* w[QH_MULTI];
    float* y[QH_MULTI];
    uint32_t wbytes[QH_MULTI];  // record count of each matrix's buffer range
    int rows[QH_MULTI];
    int tstart[QH_MULTI + 1];   // tstart[nm] = total tiles; entries past nm are INT_MAX
    // Fused prologue / epilogue of a decode step:
    //   nw != null: x is replaced by rms_norm(x) * nw (eps 1e-5) -- the kernel
    //     digitises x * nw and scales each row by rsqrt(mean(x^2) + eps), the sum
    //     of squares coming from the workgroup's own x loads (K fits one chunk);
    //   accum: y += result instead of y = result (the residual add).
    const float* nw;
    int accum;
    // Launches with NT > 1 tokens: ntok (<= NT) tokens of x, token t at x + t * ldx,
    // its results at y[m] + t * ldy[m].  Unused when NT = 1.
    int ntok, ldx;
    int ldy[QH_MULTI];
};

// The one-matrix (and SwiGLU pair) launch's arguments as leading scalars: the
// hardware preloads them into SGPRs when a wavefront starts (built with
// -amdgpu-kernarg-preload-count=16), so the first weight loads go out without
// a round trip to the kernel-argument memory (a cold miss of about 1 us; an
// aggregate argument is always read from memory).  Other multi-matrix launches
// read QhMats.
struct QhOne {
    const uint8_t* w;
    const uint8_t* w1;  // SwiGLU pairs: the up matrix (same rows and byte range as w)
    float* y;
    const float* nw;
    uint32_t wbytes;
    int rows, ntiles, accum;
};

// Tokens per launch (NT) share every weight load and B operand; the x digit
// planes, the ring of wavefront partials and the finished rows grow with NT, so
// NT > 1 keeps a shorter ring and fewer tiles per workgroup to fit 160 KB of LDS.
template <int NT>
constexpr int qh_ring() { return NT > 1 ? 2 : QH_RING; }
template <int NT>
constexpr int qh_maxt() { return NT > 2 ? 8 : (NT > 1 ? 16 : QH_MAXT); }

// LDS of one workgroup: GPW staging tiles and x digit planes per wavefront, the
// ring of wavefront partials, finished rows and the per-wavefront sums of x^2.
template <class F, int W, int GPW, int NT = 1>
constexpr int qh_mmv16_lds() {
    return W * GPW * (F::ROWS * F::RS + 16) + W * GPW * NT * QH_XG + 2 * qh_ring<NT>() * W * 16 * 4 * NT +
           qh_maxt<NT>() * 16 * 4 * NT + W * 4 * NT + (F::GRID ? 2048 : 0);
}

// The kernel body for workgroup `bid` of `nblk` working on mm's tiles (a
// launch may run two bodies of different formats side by side, see qh_mmv16_mix).
template <class F, int W, int GPW, bool X1, bool MULTI, bool PAIR, int NT = 1>
__device__ __forceinline__ void qh_mmv16_body(const QhMats& mm, const QhOne& one, const float* __restrict__ x,
                                              uint32_t row_bytes, int ngroups, unsigned char* lds, const int bid,
                                              const int nblk) {
    static_assert(!PAIR || NT == 1, "SwiGLU pairs run one token");
    constexpr int RING = qh_ring<NT>();
    constexpr int ROWS = F::ROWS, CH = F::CH;
    constexpr int NH = (ROWS * CH + 63) / 64;  // 16-byte loads per lane and group
    constexpr int RS = F::RS;                // LDS line per row
    static_assert(ROWS <= 16 && 16 * CH <= RS, "tile shape");
    constexpr int TILE = ROWS * RS + 16;  // staging tile of one group + 16 spare bytes
    // Wavefront partials of finished tiles wait in a ring of two sets of RING
    // tiles; the workgroup meets at a barrier only when a set is full.
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int ntok = NT == 1 ? 1 : mm.ntok;
    const QhBuf xb = qh_buf(x, 4u * (256u * (uint32_t)ngroups + (NT > 1 ? (uint32_t)(mm.ldx * (ntok - 1)) : 0u)));
    unsigned char* wl = lds + w * (GPW * TILE);  // GPW staging tiles of this wavefront
    // x digit planes of group t, token k at xl + (t NT + k) QH_XG
    unsigned char* xl = lds + W * GPW * TILE + w * (GPW * NT * QH_XG);
    float* red = reinterpret_cast<float*>(lds + W * GPW * TILE + W * GPW * NT * QH_XG);
    float* res = red + 2 * RING * W * 16 * NT;  // finished rows of this workgroup's tiles
    float* sqw = res + qh_maxt<NT>() * 16 * NT;  // per-wavefront sums of x^2 (fused RMS norm)
    unsigned char* gridl = reinterpret_cast<unsigned char*>(sqw + W * NT);  // IQ codebook (GRID formats)
    constexpr bool AGG = MULTI && !PAIR;  // matrices from the QhMats aggregate
    const int ntiles = AGG ? mm.tstart[QH_MULTI] : one.ntiles;
    const float* const nwp = AGG ? mm.nw : one.nw;
    // matrix of a (workgroup-uniform) tile index
    auto mat_of = [&](int tile) {
        int m = 0;
        if constexpr (PAIR) {
            m = tile & 1;
        } else if constexpr (MULTI) {
#pragma unroll
            for (int k = 1; k < QH_MULTI; k++) m += tile >= mm.tstart[k];
        }
        return m;
    };
    // Tile of matrix m's index space (PAIR: tiles alternate gate, up).
    auto local_tile = [&](int tile, int m) { return PAIR ? tile >> 1 : (MULTI ? tile - mm.tstart[m] : tile); };
    // The k-th tile of this workgroup.  PAIR (SwiGLU of two matrices): the
    // gate and up tiles of one row block follow each other, so both results
    // meet in this workgroup's LDS.
    auto wg_tile = [&](int k) -> int {
        if constexpr (PAIR) return 2 * (bid + (k >> 1) * nblk) + (k & 1);
        return bid + k * nblk;
    };
    const QhBuf wb0 = qh_buf(one.w, one.wbytes);  // the one-matrix case
    const QhBuf wb1 = qh_buf(PAIR ? one.w1 : one.w, one.wbytes);  // SwiGLU pairs: up
    const int nch = (ngroups + W * GPW - 1) / (W * GPW);

    // Slices of this lane in a tile: row rr[h], byte offset goff[h] from the
    // tile's first row, LDS offset soff[h].
    uint32_t goff[NH], soff[NH];
    int rr[NH], chs[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) {
        const int q = 64 * h + lane, r = q / CH, c = q - CH * r;
        rr[h] = q < ROWS * CH ? r : 1 << 30;
        chs[h] = c;
        goff[h] = (uint32_t)r * row_bytes + (c == CH - 1 ? F::LAST : 16u * c);
        // Lanes past ROWS * CH store into the spare bytes after the tile's last line.
        soff[h] = q < ROWS * CH ? (uint32_t)(r * RS + 16 * c) : (uint32_t)(ROWS * RS);
    }
    const int n = lane & 15, kg = lane >> 4;
    // A operand of MFMA s: digit plane n%4 of lane kg's piece in rows 4kg..4kg+2.
    // (set after the first loads are issued: see set_offsets)
    uint32_t aoff[4], xsoff[4];
    auto set_offsets = [&]() {
        const bool arow = (n >> 2) == kg && (n & 3) < 3;
        aoff[0] = arow ? 256u * (n & 3) + 16u * F::template piece<0>(kg) : QH_XG_ZERO;
        aoff[1] = arow ? 256u * (n & 3) + 16u * F::template piece<1>(kg) : QH_XG_ZERO;
        aoff[2] = arow ? 256u * (n & 3) + 16u * F::template piece<2>(kg) : QH_XG_ZERO;
        aoff[3] = arow ? 256u * (n & 3) + 16u * F::template piece<3>(kg) : QH_XG_ZERO;
        xsoff[0] = QH_XG_SUM + 4u * F::template piece<0>(kg);
        xsoff[1] = QH_XG_SUM + 4u * F::template piece<1>(kg);
        xsoff[2] = QH_XG_SUM + 4u * F::template piece<2>(kg);
        xsoff[3] = QH_XG_SUM + 4u * F::template piece<3>(kg);
    };

    // Weight loads of item (tile, ch).  Rows past out_dim and groups past in_dim
    // get offsets beyond the buffer range and read as zeros, so the load stream
    // has no branches.
    constexpr bool HALF = QhHalf<F>::value;
    // HALF: the byte shift of each slice load
    uint32_t wsa[HALF ? GPW * NH : 1];
    auto load_w = [&](int tile, int ch, qh_u32x4* wo) {
        const int g0 = ch * (W * GPW) + w * GPW;
        const int m = mat_of(tile);
        const QhBuf wb = AGG ? qh_buf(mm.w[m], mm.wbytes[m]) : (PAIR && m ? wb1 : wb0);
        const int out_dim = AGG ? mm.rows[m] : one.rows;
        if (MULTI) tile = local_tile(tile, m);
        const uint32_t base = (uint32_t)(tile * ROWS) * row_bytes;
#pragma unroll
        for (int t = 0; t < GPW; t++)
#pragma unroll
            for (int h = 0; h < NH; h++) {
                const bool ok = tile * ROWS + rr[h] < out_dim && g0 + t < ngroups;
                const uint32_t a = (ok ? base + goff[h] : 0x80000000u) + (uint32_t)F::BYTES * (uint32_t)(g0 + t);
                if constexpr (HALF) {
                    wo[t * NH + h] = qh_ld128(wb, a & ~3u);
                    wsa[t * NH + h] = a & 3u;
                } else {
                    wo[t * NH + h] = qh_ld128(wb, a);
                }
            }
    };
    // x of group t, token k -> xo[t NT + k]; tokens past ntok read as zeros.
    auto load_x = [&](int ch, float4* xo) {
        const int g0 = ch * (W * GPW) + w * GPW;
#pragma unroll
        for (int t = 0; t < GPW; t++)
#pragma unroll
            for (int k = 0; k < NT; k++) {
                // groups past in_dim read zeros too (with NT > 1 the buffer range
                // runs on into the next token's row)
                const uint32_t o = k < ntok && g0 + t < ngroups
                                       ? 1024u * (uint32_t)(g0 + t) + 16u * lane + (NT > 1 ? 4u * (uint32_t)(k * mm.ldx) : 0u)
                                       : 0x80000000u;
                const qh_u32x4 v = qh_ld128(xb, o);
                xo[t * NT + k] =
                    float4{__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w)};
            }
    };
    // Fused RMS norm (X1 only): this wavefront's sum of x^2 goes to sqw[w] and x
    // becomes x * nw.  The row scale rsqrt(mean + eps) is applied at the end.
    auto load_nw = [&](qh_u32x4* nv) {
        if constexpr (X1) {
            if (nwp) {
                const QhBuf nb = qh_buf(nwp, 4u * 256u * (uint32_t)ngroups);
#pragma unroll
                for (int t = 0; t < GPW; t++) nv[t] = qh_ld128(nb, 1024u * (uint32_t)(w * GPW + t) + 16u * lane);
            }
        }
    };
    auto norm_x = [&](float4* xo, const qh_u32x4* nv) {
        if constexpr (X1) {
            if (nwp) {
#pragma unroll
                for (int k = 0; k < NT; k++) {
                    float sq = 0.f;
#pragma unroll
                    for (int t = 0; t < GPW; t++) {
                        const qh_u32x4 v = nv[t];
                        float4& a = xo[t * NT + k];
                        sq += (a.x * a.x + a.y * a.y) + (a.z * a.z + a.w * a.w);
                        a.x *= __uint_as_float(v.x);
                        a.y *= __uint_as_float(v.y);
                        a.z *= __uint_as_float(v.z);
                        a.w *= __uint_as_float(v.w);
                    }
#pragma unroll
                    for (int o = 32; o >= 1; o >>= 1) sq += __shfl_xor(sq, o);
                    if (lane == 0) sqw[k * W + w] = sq;
                }
            }
        }
    };
    // Row scale of the fused RMS norm (1 without it); valid after a barrier.
    auto norm_scale = [&](int k) -> float {
        if constexpr (X1) {
            if (nwp) {
                float t = 0.f;
#pragma unroll
                for (int i = 0; i < W; i++) t += sqw[k * W + i];
                return rsqrtf(t / (float)(256 * ngroups) + 1e-5f);
            }
        }
        return 1.f;
    };
    // x -> digit planes in LDS.  One exponent per wavefront and chunk:
    // max|x| * 2^s < 2^22.  Returns 2^-s; `bad` turns NaN when x is not finite.
    float bad[NT];
#pragma unroll
    for (int k = 0; k < NT; k++) bad[k] = 0.f;
    auto prep_x = [&](const float4* xall, int k) -> float {
        float m = 0.f;
#pragma unroll
        for (int t = 0; t < GPW; t++) {
            const float4 xv = xall[t * NT + k];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w))));
            bad[k] += ((xv.x * 0.f + xv.y * 0.f) + (xv.z * 0.f + xv.w * 0.f));
        }
        m = qh_dpp_max(m);
        int e = 0;
        (void)frexpf(m, &e);
        int s = m > 0.f ? 22 - e : 0;
        s = s > 126 ? 126 : s;
        const float scx = ldexpf(1.0f, s);
        const uint32_t bias = 0x4B400000u - 0x808080u;
#pragma unroll
        for (int t = 0; t < GPW; t++) {
            const float4 v = xall[t * NT + k];
            unsigned char* xp = xl + (t * NT + k) * QH_XG;
            const uint32_t a0 = (__float_as_uint(fmaf(v.x, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t a1 = (__float_as_uint(fmaf(v.y, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t a2 = (__float_as_uint(fmaf(v.z, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t a3 = (__float_as_uint(fmaf(v.w, scx, 12582912.0f)) - bias) ^ 0x808080u;
            const uint32_t t01 = __builtin_amdgcn_perm(a1, a0, 0x05010400u);
            const uint32_t t23 = __builtin_amdgcn_perm(a3, a2, 0x05010400u);
            const uint32_t u01 = __builtin_amdgcn_perm(a1, a0, 0x06020602u);
            const uint32_t u23 = __builtin_amdgcn_perm(a3, a2, 0x06020602u);
            // lane holds x[256t + 4 lane .. +3] = positions 4(lane%4).. of piece lane/4.
            unsigned char* ub = xp + 4 * lane;
            *reinterpret_cast<uint32_t*>(ub) = __builtin_amdgcn_perm(t23, t01, 0x05040100u);
            *reinterpret_cast<uint32_t*>(ub + 256) = __builtin_amdgcn_perm(t23, t01, 0x07060302u);
            *reinterpret_cast<uint32_t*>(ub + 512) = __builtin_amdgcn_perm(u23, u01, 0x05040100u);
            float hs = (v.x + v.y) + (v.z + v.w);
            hs += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(hs), 0xB1, 0xF, 0xF, false));
            hs += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(hs), 0x4E, 0xF, 0xF, false));
            if ((lane & 3) == 0) *reinterpret_cast<float*>(xp + QH_XG_SUM + lane) = hs;
            if (lane == 0) *reinterpret_cast<qh_u32x4*>(xp + QH_XG_ZERO) = qh_u32x4{0, 0, 0, 0};
        }
        return ldexpf(1.0f, -s);
    };
    // Move an item's weights from registers into the GPW staging tiles.
    auto stage = [&](const qh_u32x4* wr) {
#pragma unroll
        for (int t = 0; t < GPW; t++)
#pragma unroll
            for (int h = 0; h < NH; h++) {
                qh_u32x4 v = wr[t * NH + h];
                if constexpr (HALF) {
                    // the next slice's first dword: the next lane's, lane 63's from
                    // lane 0 of the next load (past the last real slice: unused)
                    // (the slice before the last: the last starts 16 (CH - 1) - LAST bytes early,
                    // so the dword needed is its dword (16 (CH - 1) - LAST) / 4)
                    static_assert((16 * (CH - 1) - F::LAST) % 4 == 0 && 16 * (CH - 1) - F::LAST < 16, "LAST");
                    constexpr int LD = (16 * (CH - 1) - F::LAST) / 4;
                    const bool pen = chs[h] == CH - 2;
                    // DPP wave_shl:1: lane i reads lane i + 1
                    uint32_t xa = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v.x, 0x130, 0xF, 0xF, false);
                    uint32_t xb = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v[LD], 0x130, 0xF, 0xF, false);
                    if (h + 1 < NH && lane == 63) {
                        xa = (uint32_t)__builtin_amdgcn_readlane((int)wr[t * NH + h + 1].x, 0);
                        xb = (uint32_t)__builtin_amdgcn_readlane((int)wr[t * NH + h + 1][LD], 0);
                    }
                    const uint32_t x4 = pen ? xb : xa;
                    const uint32_t sh = wsa[t * NH + h];
                    v = qh_u32x4{__builtin_amdgcn_alignbyte(v.y, v.x, sh), __builtin_amdgcn_alignbyte(v.z, v.y, sh),
                                 __builtin_amdgcn_alignbyte(v.w, v.z, sh), __builtin_amdgcn_alignbyte(x4, v.w, sh)};
                }
                *reinterpret_cast<qh_u32x4*>(wl + t * TILE + soff[h]) = v;
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    // One staged item: four MFMAs per group and token, the B operands shared by
    // the tokens; out[k] = token k's partial of the lane's row.
    auto compute = [&](const float* rs, float* out) {
        float acc[NT], accm[NT];
#pragma unroll
        for (int k = 0; k < NT; k++) acc[k] = accm[k] = 0.f;
#pragma unroll
        for (int t = 0; t < GPW; t++) {
            const unsigned char* wrow = wl + t * TILE + (n < ROWS ? n : 0) * RS;
            const typename F::H hd = F::hdr(wrow, kg);
            qh_i32x4 B[4];
            F::bops(wrow, kg, hd, B, gridl);
#pragma unroll
            for (int k = 0; k < NT; k++) {
                int i0 = 0, i1 = 0, i2 = 0;
                float fm = 0.f;
                const unsigned char* xt = xl + (t * NT + k) * QH_XG;
                auto mfma = [&](auto SC) {
                    constexpr int S = decltype(SC)::value;
                    const qh_i32x4 a = *reinterpret_cast<const qh_i32x4*>(xt + aoff[S]);
                    const qh_i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, B[S], qh_i32x4{0, 0, 0, 0}, 0, 0, 0);
                    if constexpr (F::FLOAT_D) {
                        // each piece has its own f32 scale (the digit dots are exact in f32)
                        const float P = fmaf((float)D[2], 65536.0f, fmaf((float)D[1], 256.0f, (float)D[0]));
                        acc[k] = fmaf(F::template dsc<S>(hd), P, acc[k]);
                        if constexpr (F::MINS) {
                            const float xs = *reinterpret_cast<const float*>(xt + xsoff[S]);
                            fm = fmaf(F::template mnf<S>(hd), xs, fm);
                        }
                    } else {
                        const int sc = F::template scl<S>(hd, kg);
                        i0 += __mul24(sc, D[0]);
                        i1 += __mul24(sc, D[1]);
                        i2 += __mul24(sc, D[2]);
                        if constexpr (F::MINS) {
                            const float xs = *reinterpret_cast<const float*>(xt + xsoff[S]);
                            fm = fmaf((float)F::template mn<S>(hd, kg), xs, fm);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                };
                mfma(std::integral_constant<int, 0>{});
                mfma(std::integral_constant<int, 1>{});
                mfma(std::integral_constant<int, 2>{});
                mfma(std::integral_constant<int, 3>{});
                if constexpr (!F::FLOAT_D) {
                    const float P = fmaf((float)i2, 65536.0f, fmaf((float)i1, 256.0f, (float)i0));
                    acc[k] = fmaf(hd.d, P, acc[k]);
                    if constexpr (F::MINS) accm[k] = fmaf(hd.dm, fm, accm[k]);
                } else if constexpr (F::MINS) {
                    accm[k] += fm;
                }
            }
        }
#pragma unroll
        for (int k = 0; k < NT; k++) out[k] = fmaf(acc[k], rs[k], -accm[k]);
    };

    float ypre = 0.f;  // y of row threadIdx.x of the first tile (residual launches)
    auto put = [&](int d, int c, float r, int k) {  // y of row c of this workgroup's tile d, token k
        const int tile = wg_tile(d), m = mat_of(tile);
        const int row = local_tile(tile, m) * ROWS + c;
        if (c < ROWS && row < (MULTI ? mm.rows[m] : one.rows) && k < ntok) {
            float* yp = (MULTI ? mm.y[m] : one.y) + (NT > 1 ? (size_t)k * (size_t)mm.ldy[m] : 0) + row;
            // the thread that loaded this value at the start
            const bool pre = !PAIR && d == 0 && c == (int)(threadIdx.x & 15) && k == (int)(threadIdx.x >> 4);
            *yp = (MULTI ? mm.accum : one.accum) ? (pre ? ypre : *yp) + r : r;
        }
    };
    // Sum the wavefront partials of tiles d0 .. d0+cnt-1 (one set of the ring)
    // into res, or into y once the loop is over: a store inside the loop would
    // make the compiler drain all loads in flight (stores and loads share vmcnt).
    float nsc[NT];  // fused RMS-norm row scale per token, set after the first barrier
#pragma unroll
    for (int k = 0; k < NT; k++) nsc[k] = 1.f;
    auto flush = [&](int d0, int cnt, bool direct) {
        if ((int)threadIdx.x < 16 * cnt * NT) {
            const int q = (int)threadIdx.x >> 4, c = threadIdx.x & 15;
            const int k = NT > 1 ? q / cnt : 0, d = d0 + q - k * cnt;
            const float* rb = red + ((d % (2 * RING)) * NT + k) * (W * 16) + c;
            float r = 0.f;
#pragma unroll
            for (int i = 0; i < W; i++) r += rb[i * 16];
            r *= nsc[k];
            if (direct) put(d, c, r, k);
            else res[(d * NT + k) * 16 + c] = r;
        }
    };
    int tile = wg_tile(0), done = 0;
    if (tile >= ntiles) return;  // uniform over the workgroup
    // Pipeline: the registers of an item are staged into LDS as soon as they
    // arrive and then receive the loads of the next item, which stay in flight
    // while the staged item is computed.  No loaded value is copied between
    // registers (a copy would make the compiler drain every load in flight; a
    // two-set pipeline measured slower).  Items are numbered per workgroup:
    // item it = chunk it % cpt of tile it / cpt.
    const int cpt = X1 ? 1 : nch;
    auto item_tile = [&](int it) { return wg_tile(it / cpt); };
    auto item_ch = [&](int it) { return it - (it / cpt) * cpt; };
    qh_u32x4 wra[GPW * NH];
    float4 xva[GPW * NT];
    float rs[NT], tot[NT];
#pragma unroll
    for (int k = 0; k < NT; k++) rs[k] = tot[k] = 0.f;
    qh_u32x4 nv[GPW];
    // A launch's first instructions are fetched from memory (its code is
    // evicted from L2 by the weight stream of the launches before it), so the
    // first loads go out ahead of every computation they do not need (the IQ
    // formats, bound by their decode, measured better without the fence).
    if constexpr (F::GRID != 0) set_offsets();
    load_x(0, xva);
    load_nw(nv);
    load_w(tile, 0, wra);
    // Residual launches (y += W x) read the y they add to.  Thread 16k + c stores
    // row c of token k of this workgroup's first tile when the workgroup has one
    // tile, so it loads that value now, behind the first weights, and the read
    // costs no round trip at the end.
    if constexpr (!PAIR) {
        const int m = mat_of(tile), c = threadIdx.x & 15, k = (int)threadIdx.x >> 4;
        const int row = local_tile(tile, m) * ROWS + c;
        if ((MULTI ? mm.accum : one.accum) && k < ntok && c < ROWS && row < (MULTI ? mm.rows[m] : one.rows))
            ypre = (MULTI ? mm.y[m] : one.y)[(NT > 1 ? (size_t)k * (size_t)mm.ldy[m] : 0) + row];
    }
    if constexpr (F::GRID == 0) {
        __builtin_amdgcn_sched_barrier(0);
        set_offsets();
    }
    // Few tiles per workgroup: meet every RING tiles (the end-of-kernel wait
    // for the slowest wavefront is what short launches pay).  Many tiles: meet
    // at every tile (PAIR: every pair), which keeps the wavefronts on one tile's
    // rows at a time.
    const int my_tiles = PAIR ? 2 * ((ntiles / 2 - bid + nblk - 1) / nblk)
                              : (ntiles - bid + nblk - 1) / nblk;
    const int ring = my_tiles <= 2 * RING ? RING : (PAIR ? 2 : 1);
    if constexpr (F::GRID != 0) {
        const uint32_t* src = F::GRID == 1 ? qh_g_iq3s : reinterpret_cast<const uint32_t*>(qh_g_iq2xxs);
        for (int i = threadIdx.x; i < 512; i += 64 * W) reinterpret_cast<uint32_t*>(gridl)[i] = src[i];
        __syncthreads();
    }
    if constexpr (X1) {
        // x fits one chunk: digitised once, before the loop, so its registers
        // are free for the rest of the kernel
        norm_x(xva, nv);
#pragma unroll
        for (int k = 0; k < NT; k++) rs[k] = prep_x(xva, k);
    }
    int it = 0;
    auto body = [&](qh_u32x4* wr, float4* xv) -> bool {
        const int ch = item_ch(it);
        if constexpr (!X1) {
#pragma unroll
            for (int k = 0; k < NT; k++) rs[k] = prep_x(xv, k);
        }
        stage(wr);
        const int ld = it + 1;  // the item these registers load next
        if (!X1) load_x(item_ch(ld), xv);
        load_w(item_tile(ld), item_ch(ld), wr);
        {
            float part[NT];
            compute(rs, part);
#pragma unroll
            for (int k = 0; k < NT; k++) tot[k] += part[k];
        }
        const int nt = item_tile(it + 1);
        if (ch == cpt - 1) {
            // Tile finished: sum the four lanes of each column into this
            // wavefront's slot; the sum over wavefronts waits for a full set.
#pragma unroll
            for (int k = 0; k < NT; k++) {
                // a non-finite x element in any lane's share makes every row NaN
                const float bw = __ballot(!__builtin_isfinite(bad[k])) ? __builtin_nanf("") : 0.f;
                float v = tot[k] + bw;
                v += __shfl_xor(v, 16);
                v += __shfl_xor(v, 32);
                if (lane < 16) red[(((done % (2 * RING)) * NT + k) * W + w) * 16 + lane] = v;
                tot[k] = 0.f;
            }
            done++;
            if (done % ring == 0 && nt < ntiles) {
                __syncthreads();
#pragma unroll
                for (int k = 0; k < NT; k++) nsc[k] = norm_scale(k);
                flush(done - ring, ring, false);
            }
        }
        it++;
        return nt < ntiles;
    };
    while (body(wra, xva)) {
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < NT; k++) nsc[k] = norm_scale(k);
    const int last = done % ring ? done % ring : ring;
    if constexpr (PAIR) {
        // act = silu(gate) * up (qg_swiglu's expression) for every pair
        flush(done - last, last, false);
        __syncthreads();
        for (int i = threadIdx.x; i < (done >> 1) * 16; i += 64 * W) {
            const int q = i >> 4, c = i & 15, row = local_tile(wg_tile(2 * q), 0) * ROWS + c;
            if (c < ROWS && row < one.rows) {
                const float g = res[(2 * q) * 16 + c], u = res[(2 * q + 1) * 16 + c];
                one.y[row] = (g / (1.f + expf(-g))) * u;
            }
        }
        return;
    }
    // The last set goes straight to y; earlier sets wait in res.
    flush(done - last, last, true);
    for (int i = threadIdx.x; i < (done - last) * 16 * NT; i += 64 * W) put(i / (16 * NT), i & 15, res[i], (i >> 4) % NT);
}

template <class F, int W, int GPW, bool X1, bool MULTI, bool PAIR = false, int NT = 1>
__global__ __launch_bounds__(64 * W) void qh_mmv16(const float* __restrict__ x, const uint8_t* w0,
                                                   const uint8_t* w1, const float* nw0, uint32_t wbytes0, int rows0,
                                                   int ntiles0, int nblk, uint32_t row_bytes, int ngroups, float* y0,
                                                   int accum0, const QhMats mm) {
    static_assert(qh_mmv16_lds<F, W, GPW, NT>() <= 163840, "LDS");
    static_assert(MULTI || NT == 1, "one-matrix launches run one token");
    __shared__ __align__(16) unsigned char lds[qh_mmv16_lds<F, W, GPW, NT>()];
    const QhOne one = {w0, w1, y0, nw0, wbytes0, rows0, ntiles0, accum0};
    // nblk = gridDim.x, passed as a preloaded argument: gridDim comes from the
    // hidden arguments in memory, and the first loads would wait for it
    qh_mmv16_body<F, W, GPW, X1, MULTI, PAIR, NT>(mm, one, x, row_bytes, ngroups, lds, (int)blockIdx.x, nblk);
}
// The leading scalar arguments of a qh_mmv16 launch (matrices 0 and 1 of mm),
// up to the group count: 14 dwords are preloaded (the rest of the 16 user SGPRs
// hold the argument pointer), so y and the accumulate flag, needed only at the
// end, follow.
#define QH_ONE_ARGS(mm, x, grid, row_bytes, ngroups) \
    (x), (mm).w[0], (mm).w[1], (mm).nw, (mm).wbytes[0], (mm).rows[0], (mm).tstart[QH_MULTI], (grid), (row_bytes), \
        (ngroups), (mm).y[0], (mm).accum

// Two formats sharing x in one launch (a layer's q/k in Q4_K and v in Q6_K):
// workgroups below g1 run F1's body on mm1's matrices, the others F2's on mm2's.
template <class F1, class F2, int W, int GPW, bool X1, int NT = 1>
__global__ __launch_bounds__(64 * W) void qh_mmv16_mix(const QhMats mm1, const QhMats mm2, const float* __restrict__ x,
                                                       uint32_t rb1, uint32_t rb2, int ngroups, int g1) {
    constexpr int L1 = qh_mmv16_lds<F1, W, GPW, NT>(), L2 = qh_mmv16_lds<F2, W, GPW, NT>();
    __shared__ __align__(16) unsigned char lds[L1 > L2 ? L1 : L2];
    if ((int)blockIdx.x < g1)
        qh_mmv16_body<F1, W, GPW, X1, true, false, NT>(mm1, QhOne{}, x, rb1, ngroups, lds, (int)blockIdx.x, g1);
    else
        qh_mmv16_body<F2, W, GPW, X1, true, false, NT>(mm2, QhOne{}, x, rb2, ngroups, lds, (int)blockIdx.x - g1,
                                                       (int)gridDim.x - g1);
}

// nm matrices (each's weights < 2^31 bytes) in one launch.
template <class F, int W, int GPW, bool X1>
static hipError_t launch_mmv16_grid(const QhMats& mm, int nm, const float* x, int in_dim, uint32_t row_bytes,
                                     hipStream_t st, bool pair) {
    static int resident = 0;  // workgroups the device holds at once (per instantiation)
    if (!resident) {
        int dev = 0, per_cu = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, qh_mmv16<F, W, GPW, X1, false, false>,
                                                         64 * W, 0) != hipSuccess ||
            per_cu < 1)
            return hipErrorNotSupported;
        resident = per_cu * prop.multiProcessorCount;
    }
    const int tiles = mm.tstart[QH_MULTI];
    if (pair) {
        const int pairs = tiles / 2;
        int grid = pairs < resident ? pairs : resident;
        if ((pairs + grid - 1) / grid > QH_MAXT / 2) grid = (pairs + QH_MAXT / 2 - 1) / (QH_MAXT / 2);
        hipLaunchKernelGGL((qh_mmv16<F, W, GPW, X1, true, true>), dim3((unsigned)grid), dim3(64 * W), 0, st,
                           QH_ONE_ARGS(mm, x, grid, row_bytes, in_dim / 256), mm);
        return hipGetLastError();
    }
    // One workgroup per tile up to what the device holds at once (tiles go
    // round-robin, so some workgroups take one more tile than others); more
    // only when a workgroup would exceed QH_MAXT tiles.
    int grid = tiles < resident ? tiles : resident;
    if ((tiles + grid - 1) / grid > QH_MAXT) grid = (tiles + QH_MAXT - 1) / QH_MAXT;
    if (nm > 1)
        hipLaunchKernelGGL((qh_mmv16<F, W, GPW, X1, true, false>), dim3((unsigned)grid), dim3(64 * W), 0, st,
                           QH_ONE_ARGS(mm, x, grid, row_bytes, in_dim / 256), mm);
    else
        hipLaunchKernelGGL((qh_mmv16<F, W, GPW, X1, false, false>), dim3((unsigned)grid), dim3(64 * W), 0,
                           st, QH_ONE_ARGS(mm, x, grid, row_bytes, in_dim / 256), mm);
    return hipGetLastError();
}

template <class F, int W, int GPW, bool X1>
static hipError_t launch_mmv16_mats(const uint8_t* const* Ws, float* const* ys, const int* outs, int nm,
                                    const float* x, int in_dim, uint32_t row_bytes, hipStream_t st,
                                    const float* nw = nullptr, int accum = 0, bool pair = false) {
    if (nw && !X1) return hipErrorNotSupported;  // the fused norm needs all of x in one workgroup
    // SwiGLU pairs: ys[0] = silu(Ws[0] x) * (Ws[1] x), two matrices of equal rows
    if (pair && (nm != 2 || outs[0] != outs[1] || accum)) return hipErrorNotSupported;
    QhMats mm;
    int tiles = 0;
    for (int k = 0; k < QH_MULTI; k++) {
        const bool on = k < nm;
        mm.w[k] = on ? Ws[k] : nullptr;
        mm.y[k] = on ? ys[k] : nullptr;
        mm.rows[k] = on ? outs[k] : 0;
        mm.wbytes[k] = on ? (uint32_t)(((uint64_t)outs[k] * row_bytes + 3) & ~(uint64_t)3) : 0;
        mm.tstart[k] = on ? tiles : INT_MAX;
        if (on) tiles += (outs[k] + F::ROWS - 1) / F::ROWS;
    }
    mm.tstart[QH_MULTI] = tiles;
    mm.nw = nw;
    mm.accum = accum;
    if (tiles == 0) return hipSuccess;
    return launch_mmv16_grid<F, W, GPW, X1>(mm, nm, x, in_dim, row_bytes, st, pair);
}

template <class F, int W, int GPW, bool X1>
static hipError_t launch_mmv16(const uint8_t* Wt, const float* x, float* y, int in_dim, int out_dim,
                               uint32_t row_bytes, hipStream_t st) {
    // Rows are processed in chunks whose weight bytes fit a 31-bit buffer range.
    const int64_t max_rows = (((int64_t)1 << 31) - 4096) / row_bytes / F::ROWS * F::ROWS;
    if (max_rows < F::ROWS) return hipErrorNotSupported;
    for (int64_t r0 = 0; r0 < out_dim; r0 += max_rows) {
        const int rows = (int)((out_dim - r0) < max_rows ? (out_dim - r0) : max_rows);
        const uint8_t* w = Wt + (size_t)r0 * row_bytes;
        float* yy = y + r0;
        hipError_t e = launch_mmv16_mats<F, W, GPW, X1>(&w, &yy, &rows, 1, x, in_dim, row_bytes, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <class F, int W, int GPW>
static hipError_t launch_mmv16(const uint8_t* Wt, const float* x, float* y, int in_dim, int out_dim,
                               uint32_t row_bytes, hipStream_t st) {
    if (in_dim <= 256 * W * GPW) return launch_mmv16<F, W, GPW, true>(Wt, x, y, in_dim, out_dim, row_bytes, st);
    return launch_mmv16<F, W, GPW, false>(Wt, x, y, in_dim, out_dim, row_bytes, st);
}

// Launch shape: waves per workgroup W and groups per wave and chunk GPW.
// Measured on MI355X: 16 x 1 is fastest when K fits one chunk (in_dim <= 4096);
// above that 8 x 1, except Q4_K, which stays at 16 x 1 (4096 x 11008 / 14336,
// 8192 x 28672: 2-15% faster, while Q6_K and the IQ formats lose at 16 x 1).
// QUARTZ_HIP_MMV16=4|10|2|14 forces 16x1 | 8x1 | 8x2 | 14x1 (tuning).
static int qh_mmv16_variant_env() {
    static const int v = [] {
        const int k = qh_env_int("QUARTZ_HIP_MMV16", -1);
        return k == 4 || k == 10 || k == 2 || k == 14 ? k : -1;
    }();
    return v;
}
template <class F>
constexpr bool qh_mmv16_wide() {  // 16 x 1 also when K spans several chunks
    return std::is_same<F, M16Q4K>::value || std::is_same<F, M16Q4K16>::value;
}
template <class F>
constexpr bool qh_mmv16_k5() {  // Q4_K / Q5_K: 14 x 1 when K is a multiple of 14 groups
    return qh_mmv16_wide<F>() || std::is_same<F, M16Q5K>::value || std::is_same<F, M16Q5K16>::value;
}
template <class F>
static int qh_mmv16_variant(int in_dim) {
    const int v = qh_mmv16_variant_env();
    if (v >= 0) return v;
    // 14 waves when K splits into whole chunks of 14 groups (in_dim 14336: 4
    // chunks, none idle): Q4_K 4096x14336 9.95 -> 9.41 us, Q5_K 11.63 -> 10.84;
    // Q6_K loses (12.21 -> 14.47) and keeps 8 x 1
    if (in_dim > 4096 && qh_mmv16_k5<F>() && (in_dim / 256) % 14 == 0) return 14;
    return in_dim <= 4096 || qh_mmv16_wide<F>() ? 4 : 10;
}

template <class F>
static hipError_t dispatch_mmv16(const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                                 uint32_t row_bytes, hipStream_t st) {
    const int v = qh_mmv16_variant<F>(in_dim);
    switch (v) {
        case 2: return launch_mmv16<F, 8, 2>(W, x, y, in_dim, out_dim, row_bytes, st);
        case 4: return launch_mmv16<F, 16, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
        case 10: return launch_mmv16<F, 8, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
        case 14: return launch_mmv16<F, 14, 1>(W, x, y, in_dim, out_dim, row_bytes, st);
        default: return hipErrorInvalidValue;
    }
}

// Tile height: the default ROWS or 16, whichever gives the smaller
// rows-per-tile x tiles-per-CU (QUARTZ_HIP_MMV16_ROWS=16|0 forces it, tuning).
static bool qh_rows16_better(int rows, int out_dim) {
    static const int env = [] {
        const int k = qh_env_int("QUARTZ_HIP_MMV16_ROWS", -1);
        return k == 16 || k == 0 ? k : -1;
    }();
    if (env >= 0) return env == 16;
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        hipDeviceProp_t prop;
        cus = (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&prop, dev) == hipSuccess)
                  ? prop.multiProcessorCount
                  : 256;
    }
    const int64_t ra = ((int64_t)out_dim + rows - 1) / rows, rb = ((int64_t)out_dim + 15) / 16;
    return ((rb + cus - 1) / cus) * 16 < ((ra + cus - 1) / cus) * rows;
}

// Returns hipErrorNotSupported when the type/shape has no kernel here.
hipError_t qh_launch_mmv16(uint32_t type, const uint8_t* W, const float* x, float* y, int in_dim, int out_dim,
                           hipStream_t st) {
    if (in_dim % 256 || ((uintptr_t)x & 15u)) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    switch (type) {
        case QT_Q4_K:
            return qh_rows16_better(M16Q4K::ROWS, out_dim)
                       ? dispatch_mmv16<M16Q4K16>(W, x, y, in_dim, out_dim, row_bytes, st)
                       : dispatch_mmv16<M16Q4K>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q5_K:
            return qh_rows16_better(M16Q5K::ROWS, out_dim)
                       ? dispatch_mmv16<M16Q5K16>(W, x, y, in_dim, out_dim, row_bytes, st)
                       : dispatch_mmv16<M16Q5K>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q6_K:
            return in_dim <= 4096 ? dispatch_mmv16<M16Q6K>(W, x, y, in_dim, out_dim, row_bytes, st)
                                  : dispatch_mmv16<M16Q6KW>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_IQ3_S: return dispatch_mmv16<M16IQ3S>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q4_1: return dispatch_mmv16<M16Blk<1>>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q5_1: return dispatch_mmv16<M16Blk<3>>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_IQ2_XXS: return dispatch_mmv16<M16IQ2XXS>(W, x, y, in_dim, out_dim, row_bytes, st);
        case QT_Q8_0:
            return qh_rows16_better(M16Q80::ROWS, out_dim)
                       ? dispatch_mmv16<M16Q8016>(W, x, y, in_dim, out_dim, row_bytes, st)
                       : dispatch_mmv16<M16Q80>(W, x, y, in_dim, out_dim, row_bytes, st);
        default: return hipErrorNotSupported;
    }
}

// Several GEMVs sharing x (same type and in_dim) in one launch; each matrix's
// weights must fit a 31-bit buffer range.  hipErrorNotSupported otherwise.
template <class F>
static hipError_t multi_mmv16(const uint8_t* const* Ws, float* const* ys, const int* outs, int nm, const float* x,
                              int in_dim, uint32_t row_bytes, hipStream_t st, const float* nw, int accum,
                              bool pair) {
    int total = 0;
    for (int k = 0; k < nm; k++) {
        if ((int64_t)outs[k] * row_bytes >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
        total += outs[k];
    }
    const int v = qh_mmv16_variant<F>(in_dim);
    const bool x1w16 = in_dim <= 256 * 16, x1w8 = in_dim <= 256 * 8;
    (void)total;
    switch (v) {
        case 4:
            return x1w16 ? launch_mmv16_mats<F, 16, 1, true>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                         : launch_mmv16_mats<F, 16, 1, false>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case 10:
            return x1w8 ? launch_mmv16_mats<F, 8, 1, true>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                        : launch_mmv16_mats<F, 8, 1, false>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case 2:
            return in_dim <= 256 * 16 ? launch_mmv16_mats<F, 8, 2, true>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                                      : launch_mmv16_mats<F, 8, 2, false>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case 14:  // in_dim > 4096 only (K in whole chunks of 14 groups)
            return launch_mmv16_mats<F, 14, 1, false>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        default: return hipErrorInvalidValue;
    }
}

hipError_t qh_launch_mmv16_multi(uint32_t type, const uint8_t* const* Ws, float* const* ys, const int* outs, int nm,
                                 const float* x, int in_dim, hipStream_t st, const float* nw, int accum,
                                 bool pair) {
    if (nm < 1 || nm > QH_MULTI || in_dim % 256 || ((uintptr_t)x & 15u)) return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    int total = 0;
    for (int k = 0; k < nm; k++) total += outs[k];
    switch (type) {
        case QT_Q4_K:
            return qh_rows16_better(M16Q4K::ROWS, total)
                       ? multi_mmv16<M16Q4K16>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                       : multi_mmv16<M16Q4K>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_Q5_K:
            return qh_rows16_better(M16Q5K::ROWS, total)
                       ? multi_mmv16<M16Q5K16>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                       : multi_mmv16<M16Q5K>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_Q6_K:
            return in_dim <= 4096 ? multi_mmv16<M16Q6K>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                                  : multi_mmv16<M16Q6KW>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_IQ3_S: return multi_mmv16<M16IQ3S>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_Q4_1: return multi_mmv16<M16Blk<1>>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_Q5_1: return multi_mmv16<M16Blk<3>>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_IQ2_XXS: return multi_mmv16<M16IQ2XXS>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        case QT_Q8_0:
            return qh_rows16_better(M16Q80::ROWS, total)
                       ? multi_mmv16<M16Q8016>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair)
                       : multi_mmv16<M16Q80>(Ws, ys, outs, nm, x, in_dim, row_bytes, st, nw, accum, pair);
        default: return hipErrorNotSupported;
    }
}

// 2-4 tokens through the GEMV kernel: the tokens share every weight load, LDS
// stage and B operand, and each token's arithmetic is the one-token kernel's,
// so token t's result equals the GEMV of its x bit for bit.  NT = 2 or 4 (a
// third token runs in a 4-token launch with the fourth masked).
static bool qh_tokens_enabled() {
    static const int v = [] {
        return qh_env_int("QUARTZ_HIP_TOKENS", 1);
    }();
    return v != 0;
}

template <class F, int W, bool X1, int NT>
static hipError_t launch_mmv16_tok(const QhMats& mm, const float* x, int in_dim, uint32_t row_bytes, hipStream_t st) {
    static int resident = 0;
    if (!resident) {
        int dev = 0, per_cu = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, qh_mmv16<F, W, 1, X1, true, false, NT>, 64 * W, 0) !=
                hipSuccess ||
            per_cu < 1)
            return hipErrorNotSupported;
        resident = per_cu * prop.multiProcessorCount;
    }
    const int tiles = mm.tstart[QH_MULTI];
    int grid = tiles < resident ? tiles : resident;
    if ((tiles + grid - 1) / grid > qh_maxt<NT>()) grid = (tiles + qh_maxt<NT>() - 1) / qh_maxt<NT>();
    hipLaunchKernelGGL((qh_mmv16<F, W, 1, X1, true, false, NT>), dim3((unsigned)grid), dim3(64 * W), 0, st,
                       QH_ONE_ARGS(mm, x, grid, row_bytes, in_dim / 256), mm);
    return hipGetLastError();
}

template <class F>
static hipError_t tok_mmv16(int nm, const uint8_t* const* Ws, float* const* ys, const int* outs, const int* ldys,
                            const float* x, int ldx, int ntok, int in_dim, uint32_t row_bytes, int accum,
                            const float* nw, hipStream_t st) {
    QhMats mm;
    int tiles = 0;
    for (int k = 0; k < QH_MULTI; k++) {
        const bool on = k < nm;
        mm.w[k] = on ? Ws[k] : nullptr;
        mm.y[k] = on ? ys[k] : nullptr;
        mm.rows[k] = on ? outs[k] : 0;
        mm.ldy[k] = on ? ldys[k] : 0;
        mm.wbytes[k] = on ? (uint32_t)(((uint64_t)outs[k] * row_bytes + 3) & ~(uint64_t)3) : 0;
        mm.tstart[k] = on ? tiles : INT_MAX;
        if (on) tiles += (outs[k] + F::ROWS - 1) / F::ROWS;
    }
    mm.tstart[QH_MULTI] = tiles;
    mm.nw = nw;
    mm.accum = accum;
    mm.ntok = ntok;
    mm.ldx = ldx;
    if (tiles == 0) return hipSuccess;
    const bool x1 = in_dim <= 256 * 16;
    // the GEMV's launch shape, so that each token's result is bit-identical to it
    if constexpr (qh_mmv16_k5<F>())
        if (!x1 && (in_dim / 256) % 14 == 0 && qh_mmv16_variant_env() < 0)
            return ntok <= 2 ? launch_mmv16_tok<F, 14, false, 2>(mm, x, in_dim, row_bytes, st)
                             : launch_mmv16_tok<F, 14, false, 4>(mm, x, in_dim, row_bytes, st);
    if constexpr (qh_mmv16_wide<F>())
        if (!x1)
            return ntok <= 2 ? launch_mmv16_tok<F, 16, false, 2>(mm, x, in_dim, row_bytes, st)
                             : launch_mmv16_tok<F, 16, false, 4>(mm, x, in_dim, row_bytes, st);
    if (ntok <= 2)
        return x1 ? launch_mmv16_tok<F, 16, true, 2>(mm, x, in_dim, row_bytes, st)
                  : launch_mmv16_tok<F, 8, false, 2>(mm, x, in_dim, row_bytes, st);
    return x1 ? launch_mmv16_tok<F, 16, true, 4>(mm, x, in_dim, row_bytes, st)
              : launch_mmv16_tok<F, 8, false, 4>(mm, x, in_dim, row_bytes, st);
}

// Y[m][t][:] (+)= W[m] x[t] for t < ntok (x token t at x + t ldx, y token t at
// ys[m] + t ldys[m]), nm <= QH_MULTI matrices of one type sharing x.
// hipErrorNotSupported when the shape or type has no such kernel.
hipError_t qh_launch_mmv16_tokens(uint32_t type, int nm, const uint8_t* const* Ws, float* const* ys, const int* outs,
                                  const int* ldys, const float* x, int ldx, int ntok, int in_dim, int accum,
                                  hipStream_t st, const float* nw) {
    // the fused RMS norm needs a token's whole x in one workgroup (one K chunk)
    if (nw && in_dim > 256 * 16) return hipErrorNotSupported;
    if (!qh_tokens_enabled() || ntok < 2 || ntok > 4 || nm < 1 || nm > QH_MULTI || in_dim % 256 ||
        ((uintptr_t)x & 15u) || ldx % 4 || ldx < in_dim || (int64_t)ldx * (ntok - 1) + in_dim > ((int64_t)1 << 29))
        return hipErrorNotSupported;
    const uint32_t row_bytes = (uint32_t)qh_type_size(type, (size_t)in_dim);
    int total = 0;
    for (int k = 0; k < nm; k++) {
        if ((int64_t)outs[k] * row_bytes >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
        total += outs[k];
    }
    switch (type) {
        case QT_Q4_K:
            return qh_rows16_better(M16Q4K::ROWS, total)
                       ? tok_mmv16<M16Q4K16>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st)
                       : tok_mmv16<M16Q4K>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        case QT_Q5_K: return tok_mmv16<M16Q5K>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        case QT_Q6_K:
            return in_dim <= 4096 ? tok_mmv16<M16Q6K>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st)
                                  : tok_mmv16<M16Q6KW>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw,
                                                       st);
        case QT_Q8_0: return tok_mmv16<M16Q80>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        case QT_IQ3_S: return tok_mmv16<M16IQ3S>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        case QT_Q4_1: return tok_mmv16<M16Blk<1>>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        case QT_Q5_1: return tok_mmv16<M16Blk<3>>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        case QT_IQ2_XXS:
            return tok_mmv16<M16IQ2XXS>(nm, Ws, ys, outs, ldys, x, ldx, ntok, in_dim, row_bytes, accum, nw, st);
        default: return hipErrorNotSupported;
    }
}

// Two formats sharing x in one launch: matrices Ws1 (format F1) and Ws2 (F2),
// each group <= QH_MULTI matrices < 2^31 bytes.  The resident workgroups are
// split between the two bodies in proportion to their weight bytes.
// Tokens (NT > 1): ntok tokens of x at stride ldx; matrix k's results at ys[k] +
// t * ldys[k] (the one-token launch passes ldys = nullptr).
template <class F1, class F2, int W, int GPW, bool X1, int NT = 1>
static hipError_t launch_mmv16_mix(const uint8_t* const* Ws1, float* const* ys1, const int* outs1, int n1,
                                   const uint8_t* const* Ws2, float* const* ys2, const int* outs2, int n2,
                                   const float* x, int in_dim, uint32_t rb1, uint32_t rb2, const float* nw, int accum,
                                   hipStream_t st, const int* ldys1 = nullptr, const int* ldys2 = nullptr,
                                   int ldx = 0, int ntok = 1) {
    if (nw && !X1) return hipErrorNotSupported;
    static int resident = 0;
    if (!resident) {
        int dev = 0, per_cu = 0;
        hipDeviceProp_t prop;
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, qh_mmv16_mix<F1, F2, W, GPW, X1, NT>, 64 * W, 0) !=
                hipSuccess ||
            per_cu < 1)
            return hipErrorNotSupported;
        resident = per_cu * prop.multiProcessorCount;
    }
    auto fill = [&](QhMats& mm, const uint8_t* const* Ws, float* const* ys, const int* outs, int nm, uint32_t rb,
                    int rows_per_tile, const int* ldys) {
        int tiles = 0;
        mm.ntok = ntok;
        mm.ldx = ldx;
        for (int k = 0; k < QH_MULTI; k++) {
            const bool on = k < nm;
            mm.ldy[k] = on && ldys ? ldys[k] : 0;
            mm.w[k] = on ? Ws[k] : nullptr;
            mm.y[k] = on ? ys[k] : nullptr;
            mm.rows[k] = on ? outs[k] : 0;
            mm.wbytes[k] = on ? (uint32_t)(((uint64_t)outs[k] * rb + 3) & ~(uint64_t)3) : 0;
            mm.tstart[k] = on ? tiles : INT_MAX;
            if (on) tiles += (outs[k] + rows_per_tile - 1) / rows_per_tile;
        }
        mm.tstart[QH_MULTI] = tiles;
        mm.nw = nw;
        mm.accum = accum;
        return tiles;
    };
    QhMats mm1, mm2;
    const int t1 = fill(mm1, Ws1, ys1, outs1, n1, rb1, F1::ROWS, ldys1),
              t2 = fill(mm2, Ws2, ys2, outs2, n2, rb2, F2::ROWS, ldys2);
    if (t1 == 0 || t2 == 0) return hipErrorNotSupported;  // one format: the plain launch
    // Split the resident workgroups so that the side with the longer chain of
    // tiles per workgroup (tiles x tile bytes) is as short as possible.  Small
    // launches are latency-bound: a second Q6_K tile on a few workgroups costs a
    // full round, which a byte-proportional split does not see (q, k, v of an 8B
    // model: 9.0 us split by bytes, 7.1 us with v at one tile per workgroup).
    const double c1 = (double)F1::ROWS * rb1, c2 = (double)F2::ROWS * rb2;
    int g1 = 1;
    double best = 1e300;
    for (int a = 1; a < resident; a++) {
        const double cost = fmax(c1 * ((t1 + a - 1) / a), c2 * ((t2 + (resident - a) - 1) / (resident - a)));
        if (cost < best) {
            best = cost;
            g1 = a;
        }
    }
    if (resident - g1 > t2) g1 = resident - t2;  // workgroups the second side cannot use
    g1 = g1 > t1 ? t1 : g1;
    int g2 = resident - g1;
    g2 = g2 < 1 ? 1 : (g2 > t2 ? t2 : g2);
    // tiles per workgroup within the LDS ring of finished rows (more workgroups
    // than resident then, which run in a second round)
    constexpr int MAXT = qh_maxt<NT>();
    if ((t1 + g1 - 1) / g1 > MAXT) g1 = (t1 + MAXT - 1) / MAXT;
    if ((t2 + g2 - 1) / g2 > MAXT) g2 = (t2 + MAXT - 1) / MAXT;
    hipLaunchKernelGGL((qh_mmv16_mix<F1, F2, W, GPW, X1, NT>), dim3((unsigned)(g1 + g2)), dim3(64 * W), 0, st, mm1,
                       mm2, x, rb1, rb2, in_dim / 256, g1);
    return hipGetLastError();
}

template <class F1, class F2>
static hipError_t dispatch_mix_tokens(const uint8_t* const* Ws1, float* const* ys1, const int* outs1, const int* ldys1,
                                      int n1, const uint8_t* const* Ws2, float* const* ys2, const int* outs2,
                                      const int* ldys2, int n2, const float* x, int ldx, int ntok, int in_dim,
                                      uint32_t rb1, uint32_t rb2, const float* nw, int accum, hipStream_t st) {
    if (in_dim > 256 * 16) return hipErrorNotSupported;  // X1 only, as the one-token norm fusion
    if (ntok <= 2)
        return launch_mmv16_mix<F1, F2, 16, 1, true, 2>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2,
                                                        nw, accum, st, ldys1, ldys2, ldx, ntok);
    return launch_mmv16_mix<F1, F2, 16, 1, true, 4>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2, nw,
                                                    accum, st, ldys1, ldys2, ldx, ntok);
}

template <class F1, class F2>
static hipError_t dispatch_mix(const uint8_t* const* Ws1, float* const* ys1, const int* outs1, int n1,
                               const uint8_t* const* Ws2, float* const* ys2, const int* outs2, int n2, const float* x,
                               int in_dim, uint32_t rb1, uint32_t rb2, const float* nw, int accum, hipStream_t st) {
    if (in_dim <= 256 * 16)
        return launch_mmv16_mix<F1, F2, 16, 1, true>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2, nw,
                                                     accum, st);
    return launch_mmv16_mix<F1, F2, 8, 1, false>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2, nw,
                                                 accum, st);
}

// GEMVs of two matrix-core types sharing x in one launch; hipErrorNotSupported
// for other type pairs / shapes (the caller then launches per type).
hipError_t qh_launch_mmv16_mix(uint32_t t1, const uint8_t* const* Ws1, float* const* ys1, const int* outs1, int n1,
                               uint32_t t2, const uint8_t* const* Ws2, float* const* ys2, const int* outs2, int n2,
                               const float* x, int in_dim, const float* nw, int accum, hipStream_t st) {
    if (n1 < 1 || n1 > QH_MULTI || n2 < 1 || n2 > QH_MULTI || in_dim % 256 || ((uintptr_t)x & 15u) ||
        qh_mmv16_variant_env() >= 0)
        return hipErrorNotSupported;
    const uint32_t rb1 = (uint32_t)qh_type_size(t1, (size_t)in_dim), rb2 = (uint32_t)qh_type_size(t2, (size_t)in_dim);
    for (int k = 0; k < n1; k++)
        if ((int64_t)outs1[k] * rb1 >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
    for (int k = 0; k < n2; k++)
        if ((int64_t)outs2[k] * rb2 >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
    if (t1 > t2)
        return qh_launch_mmv16_mix(t2, Ws2, ys2, outs2, n2, t1, Ws1, ys1, outs1, n1, x, in_dim, nw, accum, st);
    if (t1 == QT_Q4_K && t2 == QT_Q6_K)
        return dispatch_mix<M16Q4K, M16Q6K>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2, nw, accum, st);
    if (t1 == QT_Q5_K && t2 == QT_Q6_K)
        return dispatch_mix<M16Q5K, M16Q6K>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2, nw, accum, st);
    if (t1 == QT_Q4_K && t2 == QT_Q5_K)
        return dispatch_mix<M16Q4K, M16Q5K>(Ws1, ys1, outs1, n1, Ws2, ys2, outs2, n2, x, in_dim, rb1, rb2, nw, accum, st);
    return hipErrorNotSupported;
}

// 2-4 tokens of the two-format launch (token t of x at x + t ldx, its results at
// ys[k] + t ldys[k]); each token's result is the one-token launch's bit for bit.
// X1 shapes only (in_dim <= 4096); hipErrorNotSupported otherwise.
hipError_t qh_launch_mmv16_mix_tokens(uint32_t t1, const uint8_t* const* Ws1, float* const* ys1, const int* outs1,
                                      const int* ldys1, int n1, uint32_t t2, const uint8_t* const* Ws2,
                                      float* const* ys2, const int* outs2, const int* ldys2, int n2, const float* x,
                                      int ldx, int ntok, int in_dim, const float* nw, int accum, hipStream_t st) {
    if (!qh_tokens_enabled() || ntok < 2 || ntok > 4 || n1 < 1 || n1 > QH_MULTI || n2 < 1 || n2 > QH_MULTI ||
        in_dim % 256 || ((uintptr_t)x & 15u) || (ldx & 3) || qh_mmv16_variant_env() >= 0)
        return hipErrorNotSupported;
    const uint32_t rb1 = (uint32_t)qh_type_size(t1, (size_t)in_dim), rb2 = (uint32_t)qh_type_size(t2, (size_t)in_dim);
    for (int k = 0; k < n1; k++)
        if ((int64_t)outs1[k] * rb1 >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
    for (int k = 0; k < n2; k++)
        if ((int64_t)outs2[k] * rb2 >= ((int64_t)1 << 31) - 4096) return hipErrorNotSupported;
    if (t1 > t2)
        return qh_launch_mmv16_mix_tokens(t2, Ws2, ys2, outs2, ldys2, n2, t1, Ws1, ys1, outs1, ldys1, n1, x, ldx, ntok,
                                          in_dim, nw, accum, st);
    if (t1 == QT_Q4_K && t2 == QT_Q6_K)
        return dispatch_mix_tokens<M16Q4K, M16Q6K>(Ws1, ys1, outs1, ldys1, n1, Ws2, ys2, outs2, ldys2, n2, x, ldx,
                                                   ntok, in_dim, rb1, rb2, nw, accum, st);
    if (t1 == QT_Q5_K && t2 == QT_Q6_K)
        return dispatch_mix_tokens<M16Q5K, M16Q6K>(Ws1, ys1, outs1, ldys1, n1, Ws2, ys2, outs2, ldys2, n2, x, ldx,
                                                   ntok, in_dim, rb1, rb2, nw, accum, st);
    return hipErrorNotSupported;
}
