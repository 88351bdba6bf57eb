// qh_device.h -- device-side helpers shared by every gfx950 kernel in this library.
//
// Conventions:
//  * All weight bytes are read through a raw buffer resource (V#) whose record
//    count is the byte size of the weight tensor.  Loads are 4-byte aligned
//    buffer_load_dword{,x2,x4}; an out-of-range load returns 0 instead of
//    faulting, so a window load that runs a few bytes past the end of a tensor
//    is harmless.  Byte fields that sit at 2-byte alignment (GGUF blocks of 210,
//    110, 66, 74, 82, 34, 22 or 18 bytes) are loaded as aligned dwords and
//    re-aligned in registers with v_alignbyte_b32.
//  * Wavefronts are 64 lanes; reductions use DPP row ops plus row_bcast.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define QH_DEV __device__ __forceinline__

typedef uint32_t qh_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t qh_u32x2 __attribute__((ext_vector_type(2)));

// GGML type ids (src/gguf.rs:172-191; 2/3 from the public GGUF layout).
enum : uint32_t {
    QT_F32 = 0, QT_F16 = 1, QT_Q4_0 = 2, QT_Q4_1 = 3, QT_Q5_0 = 6, QT_Q5_1 = 7, QT_Q8_0 = 8,
    QT_Q2_K = 10, QT_Q4_K = 12, QT_Q5_K = 13, QT_Q6_K = 14, QT_IQ2_XXS = 16, QT_IQ2_XS = 17,
    QT_IQ4_NL = 20, QT_IQ3_S = 21, QT_IQ2_S = 22, QT_BF16 = 30,
};

// ---------------------------------------------------------------- buffer loads

struct QhBuf {
    __amdgpu_buffer_rsrc_t rs;
};

// dword3 of a raw (untyped, stride 0) gfx9 buffer descriptor: 32-bit data format.
#define QH_RSRC_DW3 0x00020000

QH_DEV QhBuf qh_buf(const void* base, uint32_t nbytes) {
    QhBuf b;
    b.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes, QH_RSRC_DW3);
    return b;
}
QH_DEV uint32_t qh_ld32(QhBuf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(b.rs, (int)off, 0, 0);
}
QH_DEV qh_u32x2 qh_ld64(QhBuf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b64(b.rs, (int)off, 0, 0);
}
QH_DEV qh_u32x4 qh_ld128(QhBuf b, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b128(b.rs, (int)off, 0, 0);
}

// Load N dwords starting at a 4-byte aligned offset.
template <int N>
QH_DEV void qh_ldn(QhBuf b, uint32_t off, uint32_t* r) {
    int i = 0;
#pragma unroll
    for (; i + 4 <= N; i += 4) {
        qh_u32x4 v = qh_ld128(b, off + 4 * i);
        r[i] = v.x; r[i + 1] = v.y; r[i + 2] = v.z; r[i + 3] = v.w;
    }
    if constexpr (N % 4 >= 2) {
        qh_u32x2 v = qh_ld64(b, off + 4 * i);
        r[i] = v.x; r[i + 1] = v.y;
        i += 2;
    }
    if constexpr (N % 2 == 1) r[i] = qh_ld32(b, off + 4 * i);
}

// Window of N dwords starting at a 2-byte aligned offset: loads N+1 aligned
// dwords into raw[]; qh_fix() then shifts them into place.
template <int N>
QH_DEV void qh_ldwin(QhBuf b, uint32_t off, uint32_t* raw) {
    qh_ldn<N + 1>(b, off & ~3u, raw);
}
template <int N>
QH_DEV void qh_fix(const uint32_t* raw, uint32_t off, uint32_t* out) {
    const uint32_t sh = off & 3u;
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(raw[i + 1], raw[i], sh);
}

// ---------------------------------------------------------------- scalars

QH_DEV float qh_bits(uint32_t b) { return __uint_as_float(b); }

// IEEE binary16 -> f32, bit-identical to src/dequant.rs:1329-1349 for every
// pattern (subnormals exact, Inf/NaN keep their payload, no NaN quieting).
QH_DEV float qh_f16(uint32_t h) {
    h &= 0xFFFFu;
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t em = h & 0x7FFFu;
    const uint32_t normal = (em << 13) + 0x38000000u;                       // rebias 15 -> 127
    const uint32_t infnan = 0x7F800000u | ((em & 0x3FFu) << 13);
    const uint32_t sub = __float_as_uint((float)em * 0x1p-24f);            // exact: em < 2^10
    uint32_t r = em >= 0x7C00u ? infnan : (em >= 0x400u ? normal : sub);
    return qh_bits(sign | r);
}
// Hardware binary16 -> f32 (v_cvt_f32_f16): exact for every finite value
// (subnormals included); NaN payloads may be quieted.  Used for the scales in the
// GEMV kernels; the bit-exact qh_f16 is used where decoded values are returned.
QH_DEV float qh_h2f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }
QH_DEV float qh_f16_lo(uint32_t w) { return qh_h2f(w & 0xFFFFu); }
QH_DEV float qh_f16_hi(uint32_t w) { return qh_h2f(w >> 16); }

// Unsigned byte k of w as float (v_cvt_f32_ubyte{0..3}).
QH_DEV float qh_ub0(uint32_t w) { return (float)(w & 0xFFu); }
QH_DEV float qh_ub1(uint32_t w) { return (float)((w >> 8) & 0xFFu); }
QH_DEV float qh_ub2(uint32_t w) { return (float)((w >> 16) & 0xFFu); }
QH_DEV float qh_ub3(uint32_t w) { return (float)(w >> 24); }

// s += x[0..3] . bytes(w)
QH_DEV float qh_dot4u(const float* xv, uint32_t w, float s) {
    s = fmaf(xv[0], qh_ub0(w), s);
    s = fmaf(xv[1], qh_ub1(w), s);
    s = fmaf(xv[2], qh_ub2(w), s);
    s = fmaf(xv[3], qh_ub3(w), s);
    return s;
}

// Spread the low 4 bits of t (t < 16) to bit 0 of each byte.
// (t < 16 and 0x204081 < 2^24: the full-rate 24-bit multiply is exact here.)
QH_DEV uint32_t qh_spread4(uint32_t t) { return __umul24(t, 0x00204081u) & 0x01010101u; }

// Signed codebook bytes: byte j of g negated where bit j of s4 (s4 < 16) is
// set.  0x01010100 - g negates every byte at once (exact for g with no zero
// byte, true for every IQ codebook entry: the per-byte terms 256 - b are then
// all in 1..255), and one v_perm picks g's byte j (selector j) or its negation
// (j + 4).  The selector's bit 2 of byte j is bit j of s4: s4 * 0x00810204
// puts bit j at bits j + 2, j + 9, j + 16, j + 23, disjoint ranges with no
// carries, of which bit 8j + 2 is the one kept.  Five VALU operations per four
// weights with the extraction of s4 (a mask built from the bits and applied by
// xor and add took eight).
QH_DEV uint32_t qh_signbytes(uint32_t g, uint32_t s4) {
    const uint32_t sel = ((uint32_t)__umul24(s4, 0x00810204u) & 0x04040404u) | 0x03020100u;
    return __builtin_amdgcn_perm(0x01010100u - g, g, sel);
}

// ksigns_iq2xs[i] = i | parity(i) << 7  (the closed form of KSIGNS_IQ2XS).
QH_DEV uint32_t qh_ksigns(uint32_t i) { return i | ((__builtin_popcount(i) & 1u) << 7); }

// IQ pieces for the int8 matrix-core kernels: 16 consecutive weights of one
// row (half hh of 32-weight sub-block K) as signed codebook bytes b[0..3], and
// the sub-block's integer scale sc, read from a superblock staged in LDS at r
// with 16-byte slices at 16c and the last slice loaded from block byte LAST
// (so block bytes past the previous slice sit 16 (CH-1) - LAST further on).
// The B operand times sc times the format's float d is the dequantized value.
//
// IQ3_S (src/dequant.rs:1184-1237): d, qs[64], qh[8], signs[32], scales[4];
// 8-weight group l of sub-block K takes grid indices qs[8K + 2l], qs[8K + 2l +
// 1] with bits 2l, 2l+1 of qh[K] as bit 8 and signs[4K + l]; scale
// 1 + 2 * nibble K % 2 of scales[K / 2].  Last slice from byte 94: byte o >= 96
// at LDS o + 2.
QH_DEV int qh_iq3s_at(int o) { return o >= 96 ? o + 2 : o; }
QH_DEV uint32_t qh_rd16(const unsigned char* p, int o) { return *reinterpret_cast<const uint16_t*>(p + o); }
QH_DEV void qh_iq3s_piece(const unsigned char* r, int K, int hh, const uint32_t* g32, uint32_t* b, int& sc) {
    const int oq = 2 + 8 * K + 4 * hh;  // the 4 index bytes of groups 2hh, 2hh+1
    const uint32_t q = qh_rd16(r, oq) | (qh_rd16(r, oq + 2) << 16);
    const uint32_t qh = (uint32_t)r[66 + K] >> (4 * hh);
    const uint32_t sg = qh_rd16(r, qh_iq3s_at(74 + 4 * K + 2 * hh));
#pragma unroll
    for (int m = 0; m < 4; m++) {
        const uint32_t idx = ((q >> (8 * m)) & 0xFFu) | (((qh >> m) & 1u) << 8);
        b[m] = qh_signbytes(g32[idx], (sg >> (4 * m)) & 0xFu);
    }
    sc = 1 + 2 * (int)((r[qh_iq3s_at(106 + K / 2)] >> (4 * (K & 1))) & 0xFu);
}

// IQ2_XXS (src/dequant.rs:1011-1041): d, then per sub-block K 4 grid indices
// (bytes 2 + 8K ..) and a u32 (bytes 6 + 8K ..) with four 7-bit sign fields
// and the scale in bits 28-31: weight = d/8 (2 scale + 1) grid * sign.  Last
// slice from byte 50: byte o >= 64 at LDS o + 14.
QH_DEV int qh_iq2xxs_at(int o) { return o >= 64 ? o + 14 : o; }
QH_DEV void qh_iq2xxs_piece(const unsigned char* r, int K, int hh, const uint64_t* g64, uint32_t* b, int& sc) {
    const uint32_t a0 = qh_rd16(r, 2 + 8 * K + 2 * hh);  // indices of groups 2hh, 2hh+1
    const uint32_t a1 = qh_rd16(r, qh_iq2xxs_at(6 + 8 * K)) | (qh_rd16(r, qh_iq2xxs_at(8 + 8 * K)) << 16);
#pragma unroll
    for (int l = 0; l < 2; l++) {
        const uint64_t g = g64[(a0 >> (8 * l)) & 0xFFu];
        const uint32_t s8 = qh_ksigns((a1 >> (7 * (2 * hh + l))) & 127u);
        b[2 * l] = qh_signbytes((uint32_t)g, s8 & 0xFu);
        b[2 * l + 1] = qh_signbytes((uint32_t)(g >> 32), (s8 >> 4) & 0xFu);
    }
    sc = 2 * (int)(a1 >> 28) + 1;
}

// ---------------------------------------------------------------- reductions

// Full 64-lane sum; the result is valid in lane 63.
QH_DEV float qh_wave_sum63(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)); // row_half_mirror
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false)); // row_mirror
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false)); // row_bcast15
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false)); // row_bcast31
    return v;
}
