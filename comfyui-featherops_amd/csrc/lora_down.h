// Host launcher of the LoRA down-projection kernel (T = x . D^T).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace feather {

struct LoraDownArgs {
    const uint16_t* x;  // (M, K) fp16 or bf16, row-major, 16-byte aligned rows (K % 8 == 0)
    const uint16_t* d;  // (R, K) same dtype
    uint16_t* t;        // (M, R) same dtype
    int64_t M, K, R;    // R % 32 == 0
    bool bf16;
};

// Workspace the K split across workgroups can use (0: the call runs unsplit).
// Its first 64 KB are arrival counters (zero before the first call, left zero
// by every call), the rest fp32 partial tiles.
size_t lora_down_workspace_bytes(int64_t M, int64_t K, int64_t R);
// A workspace smaller than lora_down_workspace_bytes (or none) runs unsplit.
void launch_lora_down(const LoraDownArgs& a, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace feather
