// Host launchers for the quantize / layout / cast kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace feather {

// element types of weights and dequantized outputs (values shared with the C ABI)
enum WeightDtype : int { kDtypeF16 = 0, kDtypeBF16 = 1, kDtypeF32 = 2 };

struct QuantArgs {
    const void* w;            // (N, K) row-major, dtype
    int dtype;
    int64_t N, K;
    const float* ckpt_scale;  // device scalar or null (load path only)
    bool native;              // false: load path (fp32), true: patch path (weight dtype)
    uint8_t* out;             // (K/16, N, 16) e5m2 bytes
    float* scale_out;         // device scalar
    uint32_t* workspace;      // >= 1024 bytes of device memory: partial maxima (unused when scale_in is set)
    const float* scale_in;    // device scalar: use this scale instead of recalculating (native only)
    // two device words, zero on entry and left zero, for the one-pass kernel's
    // grid barrier (null: two passes); the partials then need 4 bytes per CU
    uint32_t* counters = nullptr;
    int cus = 0;              // compute units of the device (one-pass grid)
};

void launch_quantize_prepack(const QuantArgs& q, hipStream_t stream);
void launch_chunk_transpose(const uint8_t* src, uint8_t* dst, int64_t N, int64_t K, int dir, hipStream_t stream);
void launch_prepack_kn(const uint8_t* src, uint8_t* dst, int64_t K, int64_t N, hipStream_t stream);
// rne = false: round toward zero (kernel/convert.py); true: round to nearest even (torch's .to(float16))
void launch_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, bool rne, hipStream_t stream);
void launch_dequant(const uint8_t* src, const float* scale, void* dst, int64_t N, int64_t K, int dtype,
                    hipStream_t stream);

}  // namespace feather
