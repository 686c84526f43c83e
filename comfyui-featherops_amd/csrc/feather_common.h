// Shared device helpers for the gfx950 (CDNA4) FeatherOps kernels.
//
// Number formats handled here:
//   fp8 e5m2   [s:1][e:5][m:2], bias 15 -- the same exponent field and bias as
//              fp16, so widening a code to fp16 is the byte placed in the high
//              half of the 16-bit word (exact for all 256 codes, including
//              subnormals, +-inf and NaN).
//   fp8 e4m3fn [s:1][e:4][m:3], bias 7, no inf, NaN = 0x7f/0xff.
//   fp16 / bf16 outputs, rounded to nearest-even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace feather {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Workgroups of one dispatch are handed to the 8 XCDs of an MI355X
// round-robin: workgroup p runs on XCD p % 8.
constexpr int kNumXcd = 8;

__device__ __forceinline__ uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__device__ __forceinline__ float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// Returns x as computed, in an fp32 register. Placed between a multiply and a
// narrowing conversion it stops the compiler from fusing the two into one
// mixed-precision FMA: that FMA adds +0, which turns an exact -0 product
// into +0.
__device__ __forceinline__ float opaque_f32(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

__device__ __forceinline__ float half_bits_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return bits_f32(static_cast<uint32_t>(b) << 16); }

// fp32 -> fp16, round to nearest even; overflow goes to +-inf (v_cvt_f16_f32).
__device__ __forceinline__ uint16_t f32_to_half_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// fp32 -> bf16, round to nearest even; NaN becomes the canonical 0x7fc0,
// which is what torch's float -> bfloat16 conversion produces.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> bf16 bits packed (a in the low half), the same values as
// f32_to_bf16_bits: round to nearest even by one v_cvt_pk_bf16_f32, then NaN
// replaced by the canonical 0x7fc0.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float a, float b) {
    uint32_t r = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
    if (a != a) r = (r & 0xffff0000u) | 0x7fc0u;
    if (b != b) r = (r & 0x0000ffffu) | 0x7fc00000u;
    return r;
}

template <bool kBf16>
__device__ __forceinline__ uint16_t f32_to_out_bits(float f) {
    if constexpr (kBf16) return f32_to_bf16_bits(f);
    else return f32_to_half_bits(f);
}
// Two fp32 -> output bits packed (a in the low half), rounded to nearest even.
template <bool kBf16>
__device__ __forceinline__ uint32_t f32x2_to_out_bits(float a, float b) {
    if constexpr (kBf16) return f32x2_to_bf16x2_bits(a, b);
    // two scalar conversions: the packed one (v_cvt_pk_f16_f32) measured 0.5% slower on
    // the M=32768 N=13824 K=5120 epilogue
    else return static_cast<uint32_t>(f32_to_half_bits(a)) | (static_cast<uint32_t>(f32_to_half_bits(b)) << 16);
}
template <bool kBf16>
__device__ __forceinline__ float out_bits_to_f32(uint16_t b) {
    if constexpr (kBf16) return bf16_bits_to_f32(b);
    else return half_bits_to_f32(b);
}

// Widen 8 fp8 bytes (two dwords, byte j = element j) into 8 fp16 lanes,
// exactly (every fp8 value of either format is an fp16 value).
// e5m2: element j -> (byte_j << 8); one v_perm_b32 per output dword.
// e4m3fn: gfx950's OCP fp8 -> f16 conversion with scale 1 (two elements per
// instruction; subnormals exact, the two NaN codes -> NaN).
template <bool kE4m3>
__device__ __forceinline__ half8_t widen_fp8x8(uint32_t lo, uint32_t hi) {
    uint32_t w0, w1, w2, w3;
    if constexpr (!kE4m3) {
        // selector bytes: 0x0c -> 0x00, 0..3 -> bytes of the second operand
        w0 = __builtin_amdgcn_perm(0u, lo, 0x010c000cu);
        w1 = __builtin_amdgcn_perm(0u, lo, 0x030c020cu);
        w2 = __builtin_amdgcn_perm(0u, hi, 0x010c000cu);
        w3 = __builtin_amdgcn_perm(0u, hi, 0x030c020cu);
    } else {
        w0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false));
        w1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true));
        w2 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false));
        w3 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true));
    }
    uint4 v = make_uint4(w0, w1, w2, w3);
    return __builtin_bit_cast(half8_t, v);
}

// Two fp32 -> bf16 packed (a in the low half), round to nearest even, NaN
// payloads as the hardware conversion leaves them (see bf16x2_nan_seen).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_raw(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

typedef uint16_t u16x2_t __attribute__((ext_vector_type(2)));
// Running per-lane NaN detector for packed bf16 results: keep the 16-bit-wise
// maximum of (bits & 0x7fff) (one v_pk_max_u16 per word); a half above
// 0x7f80 is a NaN. Cheaper than canonicalising every pair, so the epilogues
// convert with f32x2_to_bf16x2_raw and redo a wave's values with
// f32x2_to_bf16x2_bits only when the wave saw a NaN.
__device__ __forceinline__ uint32_t bf16x2_nan_track(uint32_t acc, uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, acc),
                                                                  __builtin_bit_cast(u16x2_t, w & 0x7fff7fffu)));
}
__device__ __forceinline__ bool bf16x2_nan_seen(uint32_t acc) {
    return (acc & 0xffffu) > 0x7f80u || (acc >> 16) > 0x7f80u;
}

// v holds 8 output values (16-bit each); adds bias[0..7] elementwise in the
// output type, i.e. the exact sum rounded once to the output type. fp16: one
// packed fp16 add per pair (IEEE round to nearest even). bf16: both operands
// to fp32 (exact), the fp32 add (exact rounding of the sum to 24 bits, which
// rounds to bf16 as the exact sum would: 24 >= 2*8+2), one rounding to bf16;
// kCanonicalNaN selects torch's canonical 0x7fc0 for NaN results, otherwise
// the result words are also folded into *nan_track.
template <bool kBf16, bool kCanonicalNaN = true>
__device__ __forceinline__ void add_bias8(uint4& v, uint4 b, uint32_t* nan_track = nullptr) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (!kBf16) {
            o[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2_t, w[i]) + __builtin_bit_cast(f16x2_t, bw[i]));
        } else {
            const float lo = bf16_bits_to_f32(static_cast<uint16_t>(w[i] & 0xffffu)) +
                             bf16_bits_to_f32(static_cast<uint16_t>(bw[i] & 0xffffu));
            const float hi = bf16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16)) +
                             bf16_bits_to_f32(static_cast<uint16_t>(bw[i] >> 16));
            if constexpr (kCanonicalNaN) {
                o[i] = f32x2_to_bf16x2_bits(lo, hi);
            } else {
                o[i] = f32x2_to_bf16x2_raw(lo, hi);
                *nan_track = bf16x2_nan_track(*nan_track, o[i]);
            }
        }
    }
    v = make_uint4(o[0], o[1], o[2], o[3]);
}

// bias[0..7] packed two per word (bias needs only 2-byte alignment)
__device__ __forceinline__ uint4 load_bias8(const uint16_t* bias) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = static_cast<uint32_t>(bias[2 * i]) | (static_cast<uint32_t>(bias[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ half8_t as_half8(uint4 v) { return __builtin_bit_cast(half8_t, v); }

// An A-operand fragment of 8 activations: fp16 as stored, or bf16 converted
// to fp16 with round-to-nearest-even (overflow -> +-inf, subnormals kept), the
// same values as torch's x.to(float16) that the reference's Linear applies
// before the GEMM (comfy_feather/ops.py:88). bf16 -> fp32 is exact (a shift);
// v_cvt_pk_f16_f32 rounds two fp32 values to fp16 at once.
// Two packed bf16 values -> two packed fp16 values, round to nearest even
// (the values of torch's x.to(float16): exact widening to fp32, one rounding).
__device__ __forceinline__ uint32_t bf16x2_to_f16x2_rne(uint32_t w) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f32x2 f = {bits_f32(w << 16), bits_f32(w & 0xffff0000u)};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
}

template <bool kABf16>
__device__ __forceinline__ half8_t a_frag(uint4 v) {
    if constexpr (!kABf16) {
        return as_half8(v);
    } else {
        const uint4 o = make_uint4(bf16x2_to_f16x2_rne(v.x), bf16x2_to_f16x2_rne(v.y), bf16x2_to_f16x2_rne(v.z),
                                   bf16x2_to_f16x2_rne(v.w));
        return __builtin_bit_cast(half8_t, o);
    }
}

// D(16x16,f32) += A(16x32,f16) * B(32x16,f16). Lane l supplies A row l%16 and
// B column l%16 with 8 consecutive K slots each; lanes l and l+16*g share the
// row/column and cover slot groups g = 0..3. Any K order that is the same for
// the A and the B operand gives the same sum, which the kernels rely on.
__device__ __forceinline__ f32x4 mfma16x16x32(half8_t a, half8_t b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// The same shape on bf16 operands (8 bf16 values per lane in each uint4).
__device__ __forceinline__ f32x4 mfma16x16x32_bf16(uint4 a, uint4 b, f32x4 c) {
    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

}  // namespace feather
