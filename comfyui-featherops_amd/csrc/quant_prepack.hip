// Weight quantize-and-prepack, layout transforms and the bf16 -> fp16 cast.
//
// Quantize follows comfy_feather/quant.py:52-74 (quantize_fp8e5m2_scaled) in
// the two ways the reference calls it:
//   load path  (quant.py:116-136, make_feather_quantized_weight):
//       x = float32(w) * ckpt_scale; s = amax|x| / 57344; s==0 -> 1;
//       q = e5m2(x * (1/s))                        -- all fp32
//   patch path (quant.py:81-96,139-146, quantize_feather_weight):
//       arithmetic in the weight's own dtype T: s = float32(amax|w|) / 57344;
//       s==0 -> 1; for T = fp16 only, s = 1 / clamp(1/s, -65504, 65504);
//       inv = T(1/s); q = e5m2(T(w * inv))
// followed by the prepack of quant.py:11-13: (N, K) -> (K/16, N, 16).
// Every division is the IEEE-correctly-rounded fp32 one (hipcc's default), as
// torch's CPU division is, and the fp32 -> e5m2 conversion matches torch's
// c10 conversion: round to nearest even, |x| >= 61440 -> +-inf, NaN -> 0x7f
// with the sign bit kept.
//
// Three kernels: an amax over equal contiguous shares of the weight that
// writes one partial maximum per workgroup, a one-workgroup reduction of those partials into one 32-bit
// word, then a streaming quantize that recomputes the scale from that word in
// every thread and writes the prepacked bytes directly (16 output bytes per
// thread, 1 KB contiguous per wave). The amax pass reads the weight with
// ordinary loads, which leave it in the 256 MB MALL; the quantize pass reads it
// with nontemporal loads (they hit where it is still resident and allocate
// nothing) and writes the codes with nontemporal stores. Measured on MI355X
// with 13824 x 5120 fp16 weights rotated through 566 MB: 74 -> 68 us per
// weight; nontemporal amax loads as well make it 80 us (the quantize pass then
// finds nothing resident).
#include <cstdlib>

#include "feather_common.h"
#include "quant_prepack.h"

namespace feather {
namespace {

typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
// 16-byte load / store marked nontemporal (streamed once, not kept in the caches)
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
    const u32x4_nt t = __builtin_nontemporal_load(static_cast<const u32x4_nt*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void st_nt16(void* p, uint4 v) {
    __builtin_nontemporal_store(u32x4_nt{v.x, v.y, v.z, v.w}, static_cast<u32x4_nt*>(p));
}
constexpr float kE5m2Max = 57344.0f;
constexpr float kFp16Max = 65504.0f;

// Four fp32 -> fp8 e5m2 codes, a in the low byte: torch's c10 conversion,
// round to nearest even, |x| >= 61440 -> +-inf, NaN -> 0x7f with the sign bit
// kept. The hardware conversion (v_cvt_pk_bf8_f32, OCP e5m2, no clamp) gives
// exactly these codes for every non-NaN fp32 input (all 2^32 bit patterns
// compared on MI355X against a bit-level restatement of the rule above) and
// another NaN code, so NaN inputs are patched afterwards (kNan; callers leave
// it out where no input can be NaN).
template <bool kNan>
__device__ __forceinline__ uint32_t f32x4_to_e5m2(float a, float b, float c, float d) {
    uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false));
    w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(c, d, static_cast<int>(w), true));
    if constexpr (kNan) {
        const float v[4] = {a, b, c, d};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (__builtin_isnan(v[k]))
                w = (w & ~(0xffu << (8 * k))) | ((0x7fu | ((f32_bits(v[k]) >> 24) & 0x80u)) << (8 * k));
        }
    }
    return w;
}

template <int DT>
struct WeightType;
template <>
struct WeightType<kDtypeF16> {
    __device__ static float load(const void* p, int64_t i) { return half_bits_to_f32(static_cast<const uint16_t*>(p)[i]); }
    __device__ static float round(float f) { return half_bits_to_f32(f32_to_half_bits(f)); }
};
template <>
struct WeightType<kDtypeBF16> {
    __device__ static float load(const void* p, int64_t i) { return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]); }
    __device__ static float round(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }
};
template <>
struct WeightType<kDtypeF32> {
    __device__ static float load(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
    __device__ static float round(float f) { return f; }
};

// 16 fp16 / bf16 elements held as two 16-byte words -> fp32 (exact).
template <int DT>
__device__ __forceinline__ void decode16(const uint4 (&r)[2], float (&v)[16]) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t w[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const uint16_t lo = static_cast<uint16_t>(w[h] & 0xffffu), hi = static_cast<uint16_t>(w[h] >> 16);
            if constexpr (DT == kDtypeF16) {
                v[8 * j + 2 * h] = half_bits_to_f32(lo); v[8 * j + 2 * h + 1] = half_bits_to_f32(hi);
            } else {
                v[8 * j + 2 * h] = bf16_bits_to_f32(lo); v[8 * j + 2 * h + 1] = bf16_bits_to_f32(hi);
            }
        }
    }
}

// 16 consecutive elements starting at element index i (16-byte aligned).
template <int DT>
__device__ __forceinline__ void load16(const void* p, int64_t i, float (&v)[16]) {
    if constexpr (DT == kDtypeF32) {
        const float4* q = reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 tu = ld_nt16(&q[j]);
            const float4 t = make_float4(bits_f32(tu.x), bits_f32(tu.y), bits_f32(tu.z), bits_f32(tu.w));
            v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
        }
    } else {
        const uint4* q = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
        const uint4 r[2] = {ld_nt16(&q[0]), ld_nt16(&q[1])};
        decode16<DT>(r, v);
    }
}

// The amax pass writes one partial maximum per workgroup (plain stores: no
// atomics on one address, which serialise in L2, and nothing to clear first);
// a one-workgroup kernel reduces them into word 0, which every quantize
// workgroup reads.
constexpr int kAmaxParts = 256;
constexpr int kAmaxThreads = 1024;

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), off, 64));
        v = o > v ? o : v;
    }
    return v;
}

// amax of |x| (load path: x = w * ckpt_scale) as fp32 bits; NaN bit patterns
// compare above +inf, so a NaN anywhere yields a NaN amax as torch.amax does.
//
// The maximum is taken over the weight's own bit patterns with the sign
// cleared (for fp16, bf16 and fp32 alike that integer order is the order of
// |x|, NaNs above +inf) and scaled by |ckpt_scale| once per workgroup:
// rounding x * c is monotonic in |x| for a finite c, so max |fl(x c)| =
// fl(max|x| * |c|). A non-finite checkpoint scale (where 0 * inf = NaN
// breaks that) takes the per-element path.
template <int DT>
__device__ __forceinline__ uint32_t abs_max_words(uint4 t, uint32_t m) {
    const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        if constexpr (DT == kDtypeF32) {
            const uint32_t b = w[h] & 0x7fffffffu;
            m = b > m ? b : m;
        } else {
            const uint32_t lo = w[h] & 0x7fffu, hi = (w[h] >> 16) & 0x7fffu;
            m = lo > m ? lo : m;
            m = hi > m ? hi : m;
        }
    }
    return m;
}

template <int DT>
__device__ __forceinline__ float abs_bits_to_f32(uint32_t m) {
    if constexpr (DT == kDtypeF16) return half_bits_to_f32(static_cast<uint16_t>(m));
    else if constexpr (DT == kDtypeBF16) return bf16_bits_to_f32(static_cast<uint16_t>(m));
    else return bits_f32(m);
}

template <int DT>
__global__ __launch_bounds__(kAmaxThreads) void amax_kernel(const void* __restrict__ w, int64_t n,
                                                   const float* __restrict__ ckpt_scale, int premul,
                                                   uint32_t* __restrict__ amax_parts) {
    __shared__ uint32_t part[kAmaxThreads / 64];
    const float cs = (premul && ckpt_scale) ? ckpt_scale[0] : 1.0f;
    const bool per_element = premul && !(__builtin_fabsf(cs) <= 3.402823466e38f);  // inf or NaN scale
    uint32_t m = 0u;
    constexpr int kPerVec = DT == kDtypeF32 ? 4 : 8;  // elements per 16 bytes
    const int64_t nvec = n / kPerVec;
    const uint4* v16 = static_cast<const uint4*>(w);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    if (!per_element) {
        // native-bit maximum over this workgroup's contiguous, equal share of
        // the vectors, four 16-byte loads in flight per thread (also in the
        // last, partial round: a zero word leaves the maximum unchanged)
        const int64_t share = (nvec + gridDim.x - 1) / gridDim.x;
        const int64_t beg = static_cast<int64_t>(blockIdx.x) * share;
        const int64_t end = beg + share < nvec ? beg + share : nvec;
        for (int64_t i = beg + threadIdx.x; i < end; i += 4 * kAmaxThreads) {
            uint4 t[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                t[u] = i + u * kAmaxThreads < end ? v16[i + u * kAmaxThreads] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
            for (int u = 0; u < 4; ++u) m = abs_max_words<DT>(t[u], m);
        }
        if (blockIdx.x == 0 && threadIdx.x < n - nvec * kPerVec) {
            const int64_t t = nvec * kPerVec + threadIdx.x;
            const uint32_t b = DT == kDtypeF32 ? (static_cast<const uint32_t*>(w)[t] & 0x7fffffffu)
                                               : (static_cast<const uint16_t*>(w)[t] & 0x7fffu);
            m = b > m ? b : m;
        }
        // to |x| as fp32 (exact), then the one multiply by |ckpt_scale|
        float a = abs_bits_to_f32<DT>(m);
        if (premul) a = a * __builtin_fabsf(cs);
        m = f32_bits(a) & 0x7fffffffu;
    } else {
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
            const uint32_t b = f32_bits(WeightType<DT>::load(w, i) * cs) & 0x7fffffffu;
            m = b > m ? b : m;
        }
    }
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t r = part[0];
        for (int i = 1; i < kAmaxThreads / 64; ++i) r = part[i] > r ? part[i] : r;
        amax_parts[blockIdx.x] = r;
    }
}

// scale from amax, exactly as the reference's torch ops compute it
template <int DT>
__device__ __forceinline__ float scale_from_amax(uint32_t amax_bits, bool native) {
    float s = bits_f32(amax_bits) / kE5m2Max;
    if (s == 0.0f) s = 1.0f;
    if (native && DT == kDtypeF16) {
        float r = 1.0f / s;
        r = r < -kFp16Max ? -kFp16Max : (r > kFp16Max ? kFp16Max : r);  // NaN passes through
        s = 1.0f / r;
    }
    return s;
}

// Reduces the amax pass's partial maxima into word 0 (one workgroup).
__global__ __launch_bounds__(kAmaxParts) void amax_finalize_kernel(uint32_t* __restrict__ parts, int nparts) {
    __shared__ uint32_t red[kAmaxParts / 64];
    uint32_t m = static_cast<int>(threadIdx.x) < nparts ? parts[threadIdx.x] : 0u;
    m = wave_max_u32(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kAmaxParts / 64; ++k) m = red[k] > m ? red[k] : m;
        parts[0] = m;
    }
}

// How the codes are computed, decided once per kernel from the scale (the
// same for every thread): the patch path (arithmetic in the weight's dtype)
// or the load path (fp32 on w * ckpt_scale); on the load path with
// ckpt_scale == 1 the first multiply is left out (v * 1 == v exactly for the
// non-NaN v it is used with); NaN codes need patching only when the amax of
// the products or the reciprocal of the scale is not finite (otherwise every
// product is a finite number times a finite number: never NaN).
enum QuantMode : int { kModeLoad = 0, kModeLoadUnit = 1, kModeNative = 2, kModeNan = 4 };

struct QuantScale {
    float inv;  // T(1/s) on the patch path, 1/s on the load path
    float cs;   // ckpt_scale (load path), 1 otherwise
    int mode;
};

// amax_finite: false when unknown (a caller-given scale)
template <int DT>
__device__ __forceinline__ QuantScale quant_scale(float s, bool native, float cs, bool amax_finite) {
    QuantScale q;
    q.cs = native ? 1.0f : cs;
    q.inv = native ? WeightType<DT>::round(1.0f / s) : 1.0f / s;
    const bool nan = !amax_finite || !(__builtin_fabsf(q.inv) <= 3.402823466e38f);
    q.mode = native ? kModeNative : (q.cs == 1.0f && !nan ? kModeLoadUnit : kModeLoad);
    if (nan) q.mode |= kModeNan;
    return q;
}

template <int DT, int kMode>
__device__ __forceinline__ float scaled_elem(float v, float inv, float cs) {
    if constexpr ((kMode & kModeNative) != 0) return WeightType<DT>::round(opaque_f32(v * inv));
    else if constexpr ((kMode & kModeLoadUnit) != 0) return v * inv;
    else return (v * cs) * inv;
}

template <int DT, int kMode>
__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, float inv, float cs) {
    return f32x4_to_e5m2<(kMode & kModeNan) != 0>(scaled_elem<DT, kMode>(a, inv, cs), scaled_elem<DT, kMode>(b, inv, cs),
                                                 scaled_elem<DT, kMode>(c, inv, cs), scaled_elem<DT, kMode>(d, inv, cs));
}

// 16 elements -> 16 e5m2 codes
template <int DT, int kMode>
__device__ __forceinline__ uint4 quant16(const float (&v)[16], float inv, float cs) {
    return make_uint4(quant4<DT, kMode>(v[0], v[1], v[2], v[3], inv, cs),
                      quant4<DT, kMode>(v[4], v[5], v[6], v[7], inv, cs),
                      quant4<DT, kMode>(v[8], v[9], v[10], v[11], inv, cs),
                      quant4<DT, kMode>(v[12], v[13], v[14], v[15], inv, cs));
}

// 8 fp16 / bf16 elements held as one 16-byte word -> 8 codes (fewer live
// registers where the caller keeps many words resident)
template <int DT, int kMode>
__device__ __forceinline__ uint2 quant8(uint4 r, float inv, float cs) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint16_t bits = static_cast<uint16_t>(e & 1 ? w[e >> 1] >> 16 : w[e >> 1] & 0xffffu);
        v[e] = DT == kDtypeF16 ? half_bits_to_f32(bits) : bf16_bits_to_f32(bits);
    }
    return make_uint2(quant4<DT, kMode>(v[0], v[1], v[2], v[3], inv, cs),
                      quant4<DT, kMode>(v[4], v[5], v[6], v[7], inv, cs));
}

// calls BODY with the kernel's mode as a compile-time constant kM
#define FEATHER_QUANT_MODES(mode, BODY)                                          \
    switch (mode) {                                                               \
        case kModeLoad: { constexpr int kM = kModeLoad; BODY; } break;             \
        case kModeLoadUnit: { constexpr int kM = kModeLoadUnit; BODY; } break;     \
        case kModeNative: { constexpr int kM = kModeNative; BODY; } break;         \
        case kModeLoad | kModeNan: { constexpr int kM = kModeLoad | kModeNan; BODY; } break; \
        default: { constexpr int kM = kModeNative | kModeNan; BODY; } break;       \
    }

// grid: (ceil(K/16 / 4), ceil(N / 64)); block 256 = 64 rows (n) x 4 K-groups.
template <int DT>
__global__ __launch_bounds__(256) void quant_prepack_kernel(const void* __restrict__ w, int N, int K,
                                                            const float* __restrict__ ckpt_scale, int native,
                                                            const uint32_t* __restrict__ amax_bits,
                                                            const float* __restrict__ scale_in,
                                                            uint8_t* __restrict__ out, float* __restrict__ scale_out) {
    // scale_in: caller-supplied scale (quant.py:59-62), no recalculation and no clamp
    const uint32_t amax = scale_in ? 0u : amax_bits[0];
    const float s = scale_in ? scale_in[0] : scale_from_amax<DT>(amax, native != 0);
    if (scale_out && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) scale_out[0] = s;
    const QuantScale qs =
        quant_scale<DT>(s, native != 0, ckpt_scale ? ckpt_scale[0] : 1.0f, !scale_in && amax < 0x7f800000u);
    // thread t takes row n0 + t / 4 and K group i0 + t % 4: a wave's loads
    // cover 16 whole 128-byte row segments (16 cache lines per instruction
    // instead of 64 with one row per lane), and its stores 4 runs of 16
    // consecutive 16-byte chunks
    const int n = blockIdx.y * 64 + (threadIdx.x >> 2);
    const int i = blockIdx.x * 4 + (threadIdx.x & 3);
    if (n >= N || i >= (K >> 4)) return;

    float v[16];
    load16<DT>(w, static_cast<int64_t>(n) * K + i * 16, v);
    uint8_t* dst = out + (static_cast<int64_t>(i) * N + n) * 16;
    FEATHER_QUANT_MODES(qs.mode, st_nt16(dst, quant16<DT, kM>(v, qs.inv, qs.cs)))
}

// One-pass quantize for fp16 / bf16 weights: one workgroup per CU takes an
// equal contiguous share of the weight's blocks (64 rows x 256 elements,
// each wave load instruction two whole 512-byte row runs), keeps the first
// kResRounds of them in VGPRs (80 MB of bf16 on 256 CUs) and the next
// kResLdsBlocks in LDS (16 MB more), and reads the rest for the amax only; the workgroups exchange their partial maxima through a grid
// barrier (every workgroup's partial is stored with a device-coherent store
// and acknowledged before its arrival is counted; the partials are read only
// after all arrivals are seen), then quantize the register-held blocks, read
// the rest again and quantize those, block by block through LDS so that each
// wave stores one K group of 64 consecutive rows (1 KB contiguous in the
// (K/16, N, 16) layout). HBM traffic per element: 3 bytes for weights that fit
// the registers and LDS, 3 + 2 x (the share beyond them) otherwise, against
// the two-pass path's 5. The element arithmetic is the two-pass path's, so the
// codes are the same.
//
// The grid is one workgroup per CU, which a 1024-thread workgroup with this
// register budget fills, so every workgroup is resident at once on an idle
// device. The wait is bounded: a workgroup that does not see every arrival
// within spin_limit polls (for instance when another stream's kernels hold
// CUs) takes the amax over the whole weight by itself and goes on, so every
// workgroup finishes in any case, with the same result.
//
// Counters (words of a region that is zero on entry and left zero): arrivals
// and departures are first counted per XCD (workgroup b runs on XCD b % 8),
// each XCD's count on a line of its own, and the last workgroup of an XCD adds
// the XCD's total to the global word: 256 same-address atomics in a row would
// serialise (~10 ns each). The last workgroup to depart (all have then
// stopped reading) sets every counter back to zero. parts: one word per
// workgroup, overwritten.
constexpr int kResThreads = 1024;
constexpr int kResRounds = 10;
constexpr int kResLdsBlocks = 2;  // 64 KB of LDS beside the 67.6 KB of staging
constexpr int kResXcds = 8;
constexpr int kResLdsStride = 33;  // 16-byte chunks per LDS row: 32 + 1 pad (conflict-free column reads)
// counter words: global arrivals, global departures, then per-XCD arrivals and
// departures 64 words (256 bytes) apart
__host__ __device__ constexpr int res_arrive_word(int x) { return 64 * (1 + x); }
__host__ __device__ constexpr int res_depart_word(int x) { return 64 * (1 + kResXcds + x); }

// Chunk h (rows 0..31 or 32..63) of block blk for this thread: 16 bytes of
// row blk / nkb * 64 + 32 h + tid / 32 at elements (blk % nkb) * 256 + 8 (tid % 32)
// (K % 16 == 0, so the two chunks of a K group are valid together). Zero where
// the block runs past the weight (|0| leaves a maximum unchanged).
__device__ __forceinline__ bool chunk_valid(int blk, int h, int nkb, int N, int K) {
    const int rb = blk / nkb;
    return (blk - rb * nkb) * 256 + (threadIdx.x & 31) * 8 < K && rb * 64 + 32 * h + (threadIdx.x >> 5) < N;
}
__device__ __forceinline__ uint4 load_chunk(const void* w, int blk, int h, int nkb, int N, int K) {
    const int tid = threadIdx.x;
    const int rb = blk / nkb;
    const int k0 = (blk - rb * nkb) * 256 + (tid & 31) * 8;
    const int n = rb * 64 + 32 * h + (tid >> 5);
    return k0 < K && n < N ? ld_nt16(static_cast<const uint16_t*>(w) + static_cast<int64_t>(n) * K + k0)
                           : make_uint4(0u, 0u, 0u, 0u);
}

// amax accumulation over one chunk: over the weight's own bits (scaled by
// |ckpt_scale| once at the end), or per element over x * ckpt_scale for a
// non-finite ckpt_scale (invalid chunks skipped: 0 * inf would be NaN)
template <int DT>
__device__ __forceinline__ uint32_t amax_chunk(uint4 r, bool valid, bool per_element, float cs, uint32_t m) {
    if (!per_element) return abs_max_words<DT>(r, m);
    if (!valid) return m;
    const uint32_t wd[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint16_t bits = static_cast<uint16_t>(e & 1 ? wd[e >> 1] >> 16 : wd[e >> 1] & 0xffffu);
        const float v = DT == kDtypeF16 ? half_bits_to_f32(bits) : bf16_bits_to_f32(bits);
        const uint32_t b = f32_bits(v * cs) & 0x7fffffffu;
        m = b > m ? b : m;
    }
    return m;
}

// One block of the store phase: through LDS (the caller alternates the two
// stage buffers; the barrier of each block orders the reads of the block two
// before), wave g quantizes K group g of the block for rows tid & 63 and
// stores them as 1 KB contiguous.
template <int DT, int kMode>
__device__ __forceinline__ void store_block(uint4 c0, uint4 c1, uint4* st, int blk, int nkb, int kg, int N,
                                            const QuantScale& qs, uint8_t* __restrict__ out) {
    const int tid = threadIdx.x;
    st[(tid >> 5) * kResLdsStride + (tid & 31)] = c0;
    st[((tid >> 5) + 32) * kResLdsStride + (tid & 31)] = c1;
    __syncthreads();
    const int sg = tid >> 6, srow = tid & 63;
    const int rb = blk / nkb;
    const int g = (blk - rb * nkb) * 16 + sg;
    const int n = rb * 64 + srow;
    if (g < kg && n < N) {
        const uint2 lo = quant8<DT, kMode>(st[srow * kResLdsStride + 2 * sg], qs.inv, qs.cs);
        const uint2 hi = quant8<DT, kMode>(st[srow * kResLdsStride + 2 * sg + 1], qs.inv, qs.cs);
        st_nt16(out + (static_cast<int64_t>(g) * N + n) * 16, make_uint4(lo.x, lo.y, hi.x, hi.y));
    }
}

// The store phase: the register-held blocks, then the blocks beyond them,
// the blocks held in LDS, then the ones read again (kResStream at a time).
constexpr int kResStream = 2;
template <int DT, int kMode>
__device__ __forceinline__ void resident_store(const uint4 (&raw)[kResRounds][2], uint4 (*stage)[64 * kResLdsStride],
                                               const uint4 (*held)[2 * kResThreads], const void* w, int beg, int end,
                                               int nkb, int kg, int N, int K, const QuantScale& qs,
                                               uint8_t* __restrict__ out) {
#pragma unroll
    for (int j = 0; j < kResRounds; ++j) {
        if (beg + j >= end) return;  // uniform over the workgroup
        store_block<DT, kMode>(raw[j][0], raw[j][1], stage[j & 1], beg + j, nkb, kg, N, qs, out);
    }
#pragma unroll
    for (int e = 0; e < kResLdsBlocks; ++e) {
        const int j = kResRounds + e;
        if (beg + j >= end) return;
        store_block<DT, kMode>(held[e][threadIdx.x], held[e][kResThreads + threadIdx.x], stage[j & 1], beg + j, nkb,
                               kg, N, qs, out);
    }
    for (int blk0 = beg + kResRounds + kResLdsBlocks; blk0 < end; blk0 += kResStream) {
        uint4 t[kResStream][2];
#pragma unroll
        for (int u = 0; u < kResStream; ++u) {
            const int blk = blk0 + u < end ? blk0 + u : end - 1;
            t[u][0] = load_chunk(w, blk, 0, nkb, N, K);
            t[u][1] = load_chunk(w, blk, 1, nkb, N, K);
        }
#pragma unroll
        for (int u = 0; u < kResStream; ++u) {
            if (blk0 + u >= end) break;
            store_block<DT, kMode>(t[u][0], t[u][1], stage[(blk0 - beg + u) & 1], blk0 + u, nkb, kg, N, qs, out);
        }
    }
}

template <int DT>
__global__ __launch_bounds__(kResThreads) void quant_resident_kernel(const void* __restrict__ w, int N, int K,
                                                                     const float* __restrict__ ckpt_scale, int native,
                                                                     uint32_t* __restrict__ counters,
                                                                     uint32_t* __restrict__ parts, int spin_limit,
                                                                     uint8_t* __restrict__ out,
                                                                     float* __restrict__ scale_out) {
    static_assert(DT != kDtypeF32, "16-bit weights only");
    __shared__ __attribute__((aligned(16))) uint4 stage[2][64 * kResLdsStride];
    __shared__ __attribute__((aligned(16))) uint4 held[kResLdsBlocks][2 * kResThreads];
    __shared__ uint32_t red[kResThreads / 64];
    __shared__ int all_arrived;
    const int tid = threadIdx.x;
    const int G = static_cast<int>(gridDim.x);
    const int kg = K >> 4;                 // 16-element K groups
    const int nkb = (kg + 15) >> 4;        // 256-element K blocks
    const int nblocks = nkb * ((N + 63) >> 6);
    const int share = (nblocks + G - 1) / G;
    const int beg = static_cast<int>(blockIdx.x) * share;
    const int end = beg + share < nblocks ? beg + share : nblocks;
    const bool premul = !native;
    const float cs = (premul && ckpt_scale) ? ckpt_scale[0] : 1.0f;
    const bool per_element = premul && !(__builtin_fabsf(cs) <= 3.402823466e38f);  // inf or NaN scale

    // the first kResRounds blocks stay in registers
    uint4 raw[kResRounds][2];
#pragma unroll
    for (int j = 0; j < kResRounds; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h)
            raw[j][h] = beg + j < end ? load_chunk(w, beg + j, h, nkb, N, K) : make_uint4(0u, 0u, 0u, 0u);
    // this workgroup's maximum, in the amax kernel's terms
    uint32_t m = 0u;
    if (!per_element) {
#pragma unroll
        for (int j = 0; j < kResRounds; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) m = abs_max_words<DT>(raw[j][h], m);
    } else {
#pragma unroll
        for (int j = 0; j < kResRounds; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                if (beg + j < end) m = amax_chunk<DT>(raw[j][h], chunk_valid(beg + j, h, nkb, N, K), true, cs, m);
    }
    // the next kResLdsBlocks blocks wait in LDS (each thread keeps its own two
    // chunks: no barrier needed to read them back)
#pragma unroll
    for (int e = 0; e < kResLdsBlocks; ++e) {
        const int blk = beg + kResRounds + e;
        if (blk >= end) break;
        const uint4 t0 = load_chunk(w, blk, 0, nkb, N, K);
        const uint4 t1 = load_chunk(w, blk, 1, nkb, N, K);
        m = amax_chunk<DT>(t0, chunk_valid(blk, 0, nkb, N, K), per_element, cs, m);
        m = amax_chunk<DT>(t1, chunk_valid(blk, 1, nkb, N, K), per_element, cs, m);
        held[e][tid] = t0;
        held[e][kResThreads + tid] = t1;
    }
    // blocks beyond those: read for the amax now, again for the codes
    for (int blk = beg + kResRounds + kResLdsBlocks; blk < end; ++blk) {
        const uint4 t0 = load_chunk(w, blk, 0, nkb, N, K);
        const uint4 t1 = load_chunk(w, blk, 1, nkb, N, K);
        m = amax_chunk<DT>(t0, chunk_valid(blk, 0, nkb, N, K), per_element, cs, m);
        m = amax_chunk<DT>(t1, chunk_valid(blk, 1, nkb, N, K), per_element, cs, m);
    }
    if (!per_element) {
        float a = abs_bits_to_f32<DT>(m);
        if (premul) a = a * __builtin_fabsf(cs);
        m = f32_bits(a) & 0x7fffffffu;
    }
    m = wave_max_u32(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    const int xcd = static_cast<int>(blockIdx.x) % kResXcds;
    const uint32_t xcd_size = static_cast<uint32_t>((G - xcd + kResXcds - 1) / kResXcds);
    if (tid == 0) {
        uint32_t r = red[0];
        for (int k = 1; k < kResThreads / 64; ++k) r = red[k] > r ? red[k] : r;
        __hip_atomic_store(&parts[blockIdx.x], r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial is visible before the arrival
        if (__hip_atomic_fetch_add(&counters[res_arrive_word(xcd)], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT) == xcd_size - 1)
            __hip_atomic_fetch_add(&counters[0], xcd_size, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int ok = 0;
        for (int it = 0; it < spin_limit; ++it) {
            if (__hip_atomic_load(&counters[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >=
                static_cast<uint32_t>(G)) {
                ok = 1;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        all_arrived = ok;
    }
    __syncthreads();
    m = 0u;
    if (all_arrived) {
        if (tid < G) m = __hip_atomic_load(&parts[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        // not every workgroup arrived in time: the whole weight's amax, alone
        const int64_t nvec = static_cast<int64_t>(N) * K / 8;
        const uint4* v16 = static_cast<const uint4*>(w);
        if (!per_element) {
            for (int64_t k = tid; k < nvec; k += kResThreads) m = abs_max_words<DT>(v16[k], m);
            float a = abs_bits_to_f32<DT>(m);
            if (premul) a = a * __builtin_fabsf(cs);
            m = f32_bits(a) & 0x7fffffffu;
        } else {
            for (int64_t k = tid; k < nvec * 8; k += kResThreads) {
                const uint32_t b = f32_bits(WeightType<DT>::load(w, k) * cs) & 0x7fffffffu;
                m = b > m ? b : m;
            }
        }
    }
    m = wave_max_u32(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;  // thread 0 finished reading red[] before the barrier above
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int k = 1; k < kResThreads / 64; ++k) m = red[k] > m ? red[k] : m;
    if (tid == 0 &&
        __hip_atomic_fetch_add(&counters[res_depart_word(xcd)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            xcd_size - 1 &&
        __hip_atomic_fetch_add(&counters[1], xcd_size, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            static_cast<uint32_t>(G) - xcd_size) {
        // the last workgroup to leave: everyone has stopped polling and reading
        __hip_atomic_store(&counters[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&counters[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int x = 0; x < kResXcds; ++x) {
            __hip_atomic_store(&counters[res_arrive_word(x)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&counters[res_depart_word(x)], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }

    const float s = scale_from_amax<DT>(m, native != 0);
    if (scale_out && blockIdx.x == 0 && tid == 0) scale_out[0] = s;
    const QuantScale qs = quant_scale<DT>(s, native != 0, cs, m < 0x7f800000u);
    FEATHER_QUANT_MODES(qs.mode, (resident_store<DT, kM>(raw, stage, held, w, beg, end, nkb, kg, N, K, qs, out)))
}

// (N, K) bytes -> (K/16, N, 16) (dir 0) or back (dir 1): moves 16-byte chunks.
__global__ __launch_bounds__(256) void chunk_transpose_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                              int N, int K, int dir) {
    const int n = blockIdx.y * 64 + (threadIdx.x & 63);
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int kg = K >> 4;
    if (n >= N || i >= kg) return;
    const int64_t row_major = (static_cast<int64_t>(n) * kg + i) * 16;
    const int64_t packed = (static_cast<int64_t>(i) * N + n) * 16;
    if (dir == 0) *reinterpret_cast<uint4*>(dst + packed) = *reinterpret_cast<const uint4*>(src + row_major);
    else *reinterpret_cast<uint4*>(dst + row_major) = *reinterpret_cast<const uint4*>(src + packed);
}

// The same, block by block through LDS: a block is 64 rows x 16 K groups
// (256 bytes of each row); the row-major side moves whole 256-byte row runs
// (four per wave instruction), the packed side one K group of 64 consecutive
// rows (1 KB) per wave instruction. dir 0: (N, K) -> (K/16, N, 16); dir 1 back.
constexpr int kCtLdsStride = 17;  // 16-byte chunks per LDS row: 16 + 1 pad
template <int kDir>
__global__ __launch_bounds__(1024) void chunk_transpose_rows_kernel(const uint8_t* __restrict__ src,
                                                                    uint8_t* __restrict__ dst, int N, int K, int nkb) {
    __shared__ uint4 st[64 * kCtLdsStride];
    const int tid = threadIdx.x;
    const int rb = static_cast<int>(blockIdx.x) / nkb;
    const int kb = static_cast<int>(blockIdx.x) - rb * nkb;
    const int kg = K >> 4;
    // row-major side: row tid / 16 of the block, chunk (K group) tid % 16
    const int rrow = tid >> 4, rc = tid & 15;
    const int rn = rb * 64 + rrow;
    const int rk = kb * 256 + rc * 16;
    const bool rvalid = rn < N && rk < K;
    // packed side: K group tid / 64 of the block, row tid % 64
    const int pg = tid >> 6, prow = tid & 63;
    const int pi = kb * 16 + pg;
    const int pn = rb * 64 + prow;
    const bool pvalid = pi < kg && pn < N;
    const int64_t row_major = static_cast<int64_t>(rn) * K + rk;
    const int64_t packed = (static_cast<int64_t>(pi) * N + pn) * 16;
    if (kDir == 0) {
        if (rvalid) st[rrow * kCtLdsStride + rc] = ld_nt16(src + row_major);
        __syncthreads();
        if (pvalid) st_nt16(dst + packed, st[prow * kCtLdsStride + pg]);
    } else {
        if (pvalid) st[prow * kCtLdsStride + pg] = ld_nt16(src + packed);
        __syncthreads();
        if (rvalid) st_nt16(dst + row_major, st[rrow * kCtLdsStride + rc]);
    }
}

// (K, N) bytes -> (K/16, N, 16): P[i, n, j] = B[16 i + j, n]. One thread per
// (i, 4 columns): 16 row loads of 4 bytes, a byte transpose in registers, one
// 64-byte contiguous write.
__global__ __launch_bounds__(256) void prepack_kn_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                         int K, int N) {
    const int n4 = (blockIdx.x * 256 + threadIdx.x) * 4;
    const int i = blockIdx.y;
    if (n4 >= N) return;
    uint32_t r[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        r[j] = *reinterpret_cast<const uint32_t*>(src + static_cast<int64_t>(16 * i + j) * N + n4);
    uint4 o[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            w[q] = ((r[4 * q] >> (8 * c)) & 0xffu) | (((r[4 * q + 1] >> (8 * c)) & 0xffu) << 8) |
                   (((r[4 * q + 2] >> (8 * c)) & 0xffu) << 16) | (((r[4 * q + 3] >> (8 * c)) & 0xffu) << 24);
        }
        o[c] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    uint4* d = reinterpret_cast<uint4*>(dst + (static_cast<int64_t>(i) * N + n4) * 16);
#pragma unroll
    for (int c = 0; c < 4; ++c) d[c] = o[c];
}

// Any N: one thread per output byte.
__global__ __launch_bounds__(256) void prepack_kn_bytes_kernel(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                               int K, int N) {
    const int64_t total = static_cast<int64_t>(K) * N;
    for (int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; o < total; o += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t j = o & 15;
        const int64_t n = (o >> 4) % N;
        const int64_t i = (o >> 4) / N;
        dst[o] = src[(16 * i + j) * N + n];
    }
}

// bf16 -> fp16. kRne = false: round toward zero (v_cvt_pkrtz_f16_f32), values
// beyond the fp16 range saturate to +-65504, inf stays inf, NaN stays NaN
// (kernel/convert.py). kRne = true: round to nearest even with overflow to
// +-inf (v_cvt_pk_f16_f32), torch's x.to(float16) (comfy_feather/ops.py:88).
template <bool kRne>
__device__ __forceinline__ uint32_t bf16x2_to_fp16x2(uint32_t w) {
    const float lo = bits_f32(w << 16);
    const float hi = bits_f32(w & 0xffff0000u);
    if constexpr (kRne) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{lo, hi}), f16x2));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
    }
}

// kNT: nontemporal loads and stores, for tensors too large to stay in the
// caches for the next kernel (32768 x 5120 bf16: 133 -> 127 us on MI355X)
template <bool kRne, bool kNT>
__global__ __launch_bounds__(256) void bf16_to_fp16_kernel(const uint16_t* __restrict__ in, uint16_t* __restrict__ out,
                                                           int64_t n) {
    const int64_t nvec = n / 8;
    const uint4* in4 = reinterpret_cast<const uint4*>(in);
    uint4* out4 = reinterpret_cast<uint4*>(out);
    auto cvt = [](uint4 t) {
        return make_uint4(bf16x2_to_fp16x2<kRne>(t.x), bf16x2_to_fp16x2<kRne>(t.y), bf16x2_to_fp16x2<kRne>(t.z),
                          bf16x2_to_fp16x2<kRne>(t.w));
    };
    // each workgroup streams a contiguous, equal share of the vectors (16 KB
    // per round: four 16-byte loads in flight per thread, also in the last,
    // partial round)
    const int64_t share = (nvec + gridDim.x - 1) / gridDim.x;
    const int64_t beg = static_cast<int64_t>(blockIdx.x) * share;
    const int64_t end = beg + share < nvec ? beg + share : nvec;
    for (int64_t g = beg + threadIdx.x; g < end; g += 4 * 256) {
        uint4 t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            t[u] = g + u * 256 < end ? (kNT ? ld_nt16(&in4[g + u * 256]) : in4[g + u * 256]) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (g + u * 256 < end) {
                if (kNT) st_nt16(&out4[g + u * 256], cvt(t[u]));
                else out4[g + u * 256] = cvt(t[u]);
            }
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 7)) {
        const int64_t e = nvec * 8 + threadIdx.x;
        out[e] = static_cast<uint16_t>(bf16x2_to_fp16x2<kRne>(in[e]) & 0xffffu);
    }
}

// dequantize (K/16, N, 16) e5m2 -> (N, K) in dtype T: T(float32(q) * s),
// following quant.py:99-102 (FeatherFP8E5M2PackedLayout.dequantize); fp32
// outputs (fp16 / bf16 take dequant_rows_kernel below).
template <int DT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ src, const float* __restrict__ scale,
                                                      void* __restrict__ dst, int N, int K) {
    const int n = blockIdx.y * 64 + (threadIdx.x & 63);
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (n >= N || i >= (K >> 4)) return;
    const float s = scale[0];
    const uint4 raw = *reinterpret_cast<const uint4*>(src + (static_cast<int64_t>(i) * N + n) * 16);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint16_t h = static_cast<uint16_t>(((w[j >> 2] >> (8 * (j & 3))) & 0xffu) << 8);
        v[j] = opaque_f32(half_bits_to_f32(h) * s);  // a -0 code stays -0
    }
    const int64_t base = static_cast<int64_t>(n) * K + i * 16;
    if constexpr (DT == kDtypeF32) {
        float4* d = reinterpret_cast<float4*>(static_cast<float*>(dst) + base);
#pragma unroll
        for (int j = 0; j < 4; ++j) d[j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    } else {
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            uint32_t lo, hi;
            if constexpr (DT == kDtypeF16) { lo = f32_to_half_bits(v[2 * j]); hi = f32_to_half_bits(v[2 * j + 1]); }
            else { lo = f32_to_bf16_bits(v[2 * j]); hi = f32_to_bf16_bits(v[2 * j + 1]); }
            o[j] = lo | (hi << 16);
        }
        uint4* d = reinterpret_cast<uint4*>(static_cast<uint16_t*>(dst) + base);
        d[0] = make_uint4(o[0], o[1], o[2], o[3]);
        d[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
}

// The same for fp16 / bf16 outputs, block by block through LDS: a block is 64
// rows x 256 elements (16 K groups); wave g reads K group g of the block's 64
// rows (1 KB contiguous in the (K/16, N, 16) layout), converts it and puts
// each row's 16 values into LDS; then each wave writes two whole 512-byte row
// runs of the (N, K) output. Codes and output are streamed once (nontemporal
// accesses). Element arithmetic as dequant_kernel. 13824 x 5120 -> fp16 on
// MI355X: 41.6 us (5.1 TB/s on 3 B per element) against 78 us for
// dequant_kernel's one-row-per-lane 32-byte writes (45.8 us with ordinary
// loads and stores).
constexpr int kDqLdsStride = 33;  // 16-byte chunks per LDS row: 32 + 1 pad
template <int DT>
__global__ __launch_bounds__(1024) void dequant_rows_kernel(const uint8_t* __restrict__ src,
                                                            const float* __restrict__ scale,
                                                            uint16_t* __restrict__ dst, int N, int K, int nkb) {
    static_assert(DT != kDtypeF32, "16-bit outputs");
    __shared__ __attribute__((aligned(16))) uint4 st[64 * kDqLdsStride];
    const int tid = threadIdx.x;
    const int blk = blockIdx.x;
    const int rb = blk / nkb;
    const int kb = blk - rb * nkb;
    const int kg = K >> 4;
    const float s = scale[0];
    {
        const int g = tid >> 6;     // K group within the block
        const int row = tid & 63;   // row within the block
        const int i = kb * 16 + g;
        const int n = rb * 64 + row;
        if (i < kg && n < N) {
            const uint8_t* p = src + (static_cast<int64_t>(i) * N + n) * 16;
            const uint4 raw = ld_nt16(p);
            const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
            uint32_t o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                uint32_t half[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int q = 2 * j + e;
                    const uint16_t h = static_cast<uint16_t>(((w[q >> 2] >> (8 * (q & 3))) & 0xffu) << 8);
                    const float v = opaque_f32(half_bits_to_f32(h) * s);  // a -0 code stays -0
                    half[e] = DT == kDtypeF16 ? f32_to_half_bits(v) : f32_to_bf16_bits(v);
                }
                o[j] = half[0] | (half[1] << 16);
            }
            st[row * kDqLdsStride + 2 * g] = make_uint4(o[0], o[1], o[2], o[3]);
            st[row * kDqLdsStride + 2 * g + 1] = make_uint4(o[4], o[5], o[6], o[7]);
        }
    }
    __syncthreads();
    const int c = tid & 31;        // 16-byte chunk of the row's 512-byte run
    const int k = kb * 256 + c * 8;  // first element (K % 16 == 0: the chunk is whole when it starts inside)
    if (k < K) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int row = (tid >> 5) + 32 * h;
            const int n = rb * 64 + row;
            if (n < N) {
                uint16_t* q = dst + static_cast<int64_t>(n) * K + k;
                st_nt16(q, st[row * kDqLdsStride + c]);
            }
        }
    }
}

int grid_for(int64_t work, int per_block, int cap) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return static_cast<int>(g);
}

// FEATHEROPS_QUANT_RESIDENT=0 keeps the two-pass path everywhere;
// FEATHEROPS_QUANT_SPIN sets the grid barrier's poll limit (tests force the
// fallback with 0).
bool resident_enabled() {
    const char* e = std::getenv("FEATHEROPS_QUANT_RESIDENT");
    return !(e && e[0] == '0');
}

int resident_spin_limit() {
    const char* e = std::getenv("FEATHEROPS_QUANT_SPIN");
    return e ? std::atoi(e) : 4096;
}

template <int DT>
bool launch_quant_resident(const QuantArgs& q, hipStream_t stream) {
    if (!q.counters || q.scale_in || q.cus <= 0 || q.cus > kResThreads || !resident_enabled()) return false;
    const int64_t nblocks = ((q.K / 16 + 15) / 16) * ((q.N + 63) / 64);
    if (nblocks >= (int64_t(1) << 30)) return false;  // block indices in int
    hipLaunchKernelGGL((quant_resident_kernel<DT>), dim3(q.cus), dim3(kResThreads), 0, stream, q.w,
                       static_cast<int>(q.N), static_cast<int>(q.K), q.ckpt_scale, q.native ? 1 : 0, q.counters,
                       q.workspace, resident_spin_limit(), q.out, q.scale_out);
    return true;
}

template <int DT>
void launch_quant(const QuantArgs& q, hipStream_t stream) {
    const int64_t n = q.N * q.K;
    const bool premul = !q.native;
    // amax workgroups: one round of four 16-byte loads per thread covers
    // 1024 * 4 * 16 bytes; at most kAmaxParts workgroups, looping over the rest
    const int64_t round_elems = static_cast<int64_t>(kAmaxThreads) * 4 * (DT == kDtypeF32 ? 4 : 8);
    const int nparts = q.scale_in ? 0 : grid_for(n, static_cast<int>(round_elems), kAmaxParts);
    if (!q.scale_in) {
        hipLaunchKernelGGL((amax_kernel<DT>), dim3(nparts), dim3(kAmaxThreads), 0, stream, q.w, n, q.ckpt_scale,
                           premul ? 1 : 0, q.workspace);
        hipLaunchKernelGGL(amax_finalize_kernel, dim3(1), dim3(kAmaxParts), 0, stream, q.workspace, nparts);
    }
    const dim3 grid(static_cast<uint32_t>((q.K / 16 + 3) / 4), static_cast<uint32_t>((q.N + 63) / 64));
    hipLaunchKernelGGL((quant_prepack_kernel<DT>), grid, dim3(256), 0, stream, q.w, static_cast<int>(q.N),
                       static_cast<int>(q.K), q.ckpt_scale, q.native ? 1 : 0, q.workspace, q.scale_in, q.out,
                       q.scale_out);
}

}  // namespace

void launch_quantize_prepack(const QuantArgs& q, hipStream_t stream) {
    switch (q.dtype) {
        case kDtypeF16:
            if (!launch_quant_resident<kDtypeF16>(q, stream)) launch_quant<kDtypeF16>(q, stream);
            break;
        case kDtypeBF16:
            if (!launch_quant_resident<kDtypeBF16>(q, stream)) launch_quant<kDtypeBF16>(q, stream);
            break;
        default: launch_quant<kDtypeF32>(q, stream); break;
    }
}

void launch_chunk_transpose(const uint8_t* src, uint8_t* dst, int64_t N, int64_t K, int dir, hipStream_t stream) {
    const int nkb = static_cast<int>((K / 16 + 15) / 16);
    const int64_t nblocks = static_cast<int64_t>(nkb) * ((N + 63) / 64);
    if (nblocks < (int64_t(1) << 31)) {
        const dim3 g(static_cast<uint32_t>(nblocks));
        if (dir == 0)
            hipLaunchKernelGGL(chunk_transpose_rows_kernel<0>, g, dim3(1024), 0, stream, src, dst, static_cast<int>(N),
                               static_cast<int>(K), nkb);
        else
            hipLaunchKernelGGL(chunk_transpose_rows_kernel<1>, g, dim3(1024), 0, stream, src, dst, static_cast<int>(N),
                               static_cast<int>(K), nkb);
        return;
    }
    const dim3 grid(static_cast<uint32_t>((K / 16 + 3) / 4), static_cast<uint32_t>((N + 63) / 64));
    hipLaunchKernelGGL(chunk_transpose_kernel, grid, dim3(256), 0, stream, src, dst, static_cast<int>(N),
                       static_cast<int>(K), dir);
}

void launch_prepack_kn(const uint8_t* src, uint8_t* dst, int64_t K, int64_t N, hipStream_t stream) {
    if (N % 4 == 0 && (reinterpret_cast<uintptr_t>(src) & 3u) == 0) {
        const dim3 grid(static_cast<uint32_t>((N / 4 + 255) / 256), static_cast<uint32_t>(K / 16));
        hipLaunchKernelGGL(prepack_kn_kernel, grid, dim3(256), 0, stream, src, dst, static_cast<int>(K),
                           static_cast<int>(N));
    } else {
        hipLaunchKernelGGL(prepack_kn_bytes_kernel, dim3(grid_for(K * N, 256, 8192)), dim3(256), 0, stream, src, dst,
                           static_cast<int>(K), static_cast<int>(N));
    }
}

void launch_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, bool rne, hipStream_t stream) {
    const dim3 grid(grid_for(n / 32, 256, 8192));
    // at least 128 MB in: the output would not survive in the 256 MB MALL for the next kernel anyway
    const bool nt = n >= (int64_t(64) << 20);
    if (rne) {
        if (nt) hipLaunchKernelGGL((bf16_to_fp16_kernel<true, true>), grid, dim3(256), 0, stream, in, out, n);
        else hipLaunchKernelGGL((bf16_to_fp16_kernel<true, false>), grid, dim3(256), 0, stream, in, out, n);
    } else {
        if (nt) hipLaunchKernelGGL((bf16_to_fp16_kernel<false, true>), grid, dim3(256), 0, stream, in, out, n);
        else hipLaunchKernelGGL((bf16_to_fp16_kernel<false, false>), grid, dim3(256), 0, stream, in, out, n);
    }
}

void launch_dequant(const uint8_t* src, const float* scale, void* dst, int64_t N, int64_t K, int dtype,
                    hipStream_t stream) {
    if (dtype != kDtypeF32) {
        const int nkb = static_cast<int>((K / 16 + 15) / 16);
        const int64_t nblocks = static_cast<int64_t>(nkb) * ((N + 63) / 64);
        if (nblocks < (int64_t(1) << 31)) {
            const dim3 g(static_cast<uint32_t>(nblocks));
            uint16_t* d = static_cast<uint16_t*>(dst);
            const int n32 = static_cast<int>(N), k32 = static_cast<int>(K);
            if (dtype == kDtypeF16)
                hipLaunchKernelGGL((dequant_rows_kernel<kDtypeF16>), g, dim3(1024), 0, stream, src, scale, d, n32, k32, nkb);
            else
                hipLaunchKernelGGL((dequant_rows_kernel<kDtypeBF16>), g, dim3(1024), 0, stream, src, scale, d, n32, k32, nkb);
            return;
        }
    }
    const dim3 grid(static_cast<uint32_t>((K / 16 + 3) / 4), static_cast<uint32_t>((N + 63) / 64));
    switch (dtype) {
        case kDtypeF16:
            hipLaunchKernelGGL((dequant_kernel<kDtypeF16>), grid, dim3(256), 0, stream, src, scale, dst,
                               static_cast<int>(N), static_cast<int>(K));
            break;
        case kDtypeBF16:
            hipLaunchKernelGGL((dequant_kernel<kDtypeBF16>), grid, dim3(256), 0, stream, src, scale, dst,
                               static_cast<int>(N), static_cast<int>(K));
            break;
        default:
            hipLaunchKernelGGL((dequant_kernel<kDtypeF32>), grid, dim3(256), 0, stream, src, scale, dst,
                               static_cast<int>(N), static_cast<int>(K));
            break;
    }
}

}  // namespace feather
