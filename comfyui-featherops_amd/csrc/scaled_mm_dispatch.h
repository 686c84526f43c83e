// Host-side description of one scaled_mm call and the gfx950 kernel variants
// that can serve it.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace feather {

struct MmArgs {
    const uint16_t* a;       // (M, K) fp16 (or bf16 when a_bf16), row-major
    const uint8_t* b;        // (K/16, N, 16) fp8 bytes
    const float* scale;      // device scalar, read when has_scale
    const uint16_t* bias;    // (N,) in the output type, read when has_bias
    uint16_t* c;             // (M, N) fp16 / bf16, row-major
    int64_t M, N, K;
    int has_scale, has_bias;
    bool out_bf16;
    bool b_e4m3;
    bool a_bf16;             // activations are bf16 (converted to fp16 in the kernel; e5m2 weights only)
    int group_m;             // tile raster group height (0 = default)
    int smallm_min_groups;   // small-M: workgroup count the K split aims for (0 = default)
    // rank-R epilogue update C += T . U^T (LDS tiles only): T (M, R), U (N, R)
    const uint16_t* lora_t = nullptr;
    const uint16_t* lora_u = nullptr;
    int64_t lora_rank = 0;
    int lora_dtype = 0;      // 0 none, 1 fp16 factors, 2 bf16 factors
};

// Kernel variants. Values are stable: the Python autotuner de-duplicates
// reference configs by the id they map to.
enum KernelId : int {
    kKernelNone = 0,
    kTile256x256 = 1,
    kTile256x128 = 2,
    kTile128x256 = 3,
    kTile128x128 = 4,
    kTile64x128 = 5,
    kTile64x64 = 6,
    kSmallM = 10,  // M <= 64: K split inside the workgroup (and across workgroups with a workspace), 16- or 64-column strips
    // LDS-DMA pipelined tiles (K % 64 == 0)
    kLds256x256 = 20,  // both 256 x 256 tuples (2,4,4,8,4) and (4,2,4,4,8)
    kLds256x128 = 22,
    kLds128x256 = 23,
    kLds128x128 = 24,
    kLds256x192 = 25,
    kLds128x384 = 26,
    // LDS-DMA tiles with a K split across workgroups (small shapes)
    kLdsSk64x64 = 30,
    kLdsSk64x128 = 31,
    kLdsSk32x128 = 34,
};

// Every launcher returns false, and launches nothing, for a variant it does not
// have (bf16 activations are served by the split-K LDS tiles and the small-M
// kernel with e5m2 weights only).
bool launch_tile_kernel(int kernel_id, const MmArgs& p, hipStream_t stream);
// K-split workspace layout, shared by the small-M kernel and the split-K LDS
// tiles: a fixed region of arrival counters (one u32 per output strip or tile)
// that nothing else ever writes, then the fp32 partials. The counter region
// must be zero before the first call and every call leaves it zero again, so
// one workspace serves calls of any shapes in any order (a counter region
// sized per call would overlap an earlier call's partials). A split that would
// need more counters than the region holds is not taken.
constexpr int64_t kWorkspaceCounters = 16384;
constexpr size_t kWorkspaceCounterBytes = static_cast<size_t>(kWorkspaceCounters) * 4;  // 64 KB

// Small-M kernel. With a workspace of at least smallm_workspace_bytes() it
// also splits K across workgroups; without one it splits K inside each
// workgroup only.
bool launch_smallm_kernel(const MmArgs& p, void* workspace, size_t workspace_bytes, hipStream_t stream);
size_t smallm_workspace_bytes(int64_t M, int64_t N, int64_t K, int target_groups);
int smallm_ksplit(int64_t M, int64_t N, int64_t K, int target_groups);
bool launch_lds_kernel(int kernel_id, const MmArgs& p, hipStream_t stream);

struct SplitKPlan {
    int kernel_id;          // 0: not applicable
    int ksplit;
    int tiles;
    size_t counter_bytes;   // the fixed counter region (kWorkspaceCounterBytes) when ksplit > 1
    size_t workspace_bytes; // counter region + ksplit fp32 partial tiles per output tile
    int stages;             // LDS stage ring depth of the default schedule (5 or 6)
};
SplitKPlan lds_splitk_plan(int64_t M, int64_t N, int64_t K, int target);
// Same workspace contract as launch_smallm_kernel.
bool launch_lds_splitk(const MmArgs& p, void* workspace, size_t workspace_bytes, hipStream_t stream);

}  // namespace feather
