// extern "C" entry points of libfeatherops_amd.so (declared in
// include/featherops_amd.h). Validation that needs only sizes and pointers
// lives here; dtype/stride checks of torch tensors live in the Python layer.
#include <stdint.h>
#include <stdlib.h>

#include <mutex>

#include "featherops_amd.h"
#include "lora_down.h"
#include "quant_prepack.h"
#include "scaled_mm_dispatch.h"

namespace {

using feather::KernelId;

struct Cfg {
    int wm, wn, u, rm, rn;
};

// Reference configurations (kernel/hip/hip_kernel.py:60-89, hip_kernel.cu:603-630)
// followed by five gfx950 tiles the reference has no tuple for.
constexpr Cfg kConfigs[] = {
    {1, 1, 2, 1, 2}, {1, 1, 4, 1, 2}, {1, 2, 2, 1, 2}, {1, 2, 4, 1, 2}, {1, 4, 2, 1, 2}, {1, 4, 4, 1, 2},
    {1, 8, 2, 1, 2}, {1, 8, 4, 1, 2}, {1, 1, 2, 2, 2}, {1, 1, 4, 2, 2}, {1, 1, 2, 4, 4}, {1, 1, 4, 4, 4},
    {1, 2, 2, 2, 2}, {1, 2, 4, 2, 2}, {2, 1, 2, 2, 2}, {2, 1, 4, 2, 2}, {1, 4, 2, 4, 2}, {1, 4, 4, 4, 2},
    {1, 8, 2, 8, 2}, {1, 8, 4, 8, 2}, {2, 2, 2, 4, 4}, {2, 2, 4, 4, 4}, {2, 4, 2, 4, 2}, {2, 4, 4, 4, 2},
    {2, 4, 2, 4, 4}, {2, 4, 4, 4, 4}, {4, 2, 2, 2, 4}, {4, 2, 4, 2, 4},
    {2, 4, 4, 8, 4}, {4, 2, 4, 4, 4}, {4, 2, 4, 4, 8}, {2, 4, 4, 8, 3}, {2, 4, 4, 4, 6},
};

bool known_config(int wm, int wn, int u, int rm, int rn) {
    for (const Cfg& c : kConfigs)
        if (c.wm == wm && c.wn == wn && c.u == u && c.rm == rm && c.rn == rn) return true;
    return false;
}

// The tuple picks the output tile (BlockM x BlockN, capped at 256); the
// LDS-DMA pipeline serves K % 64 == 0, the register-staged tile the rest.
// Shapes too small to fill the GPU with those tiles are routed first (see
// splitk_route).
int tile_kernel_for(int64_t M, int64_t K, int wm, int wn, int rm, int rn) {
    if (M <= 64) return feather::kSmallM;
    const int bm = 16 * wm * rm;
    const int bn = 16 * wn * rn;
    const bool lds = K % 64 == 0;
    if (bm >= 256 && bn == 192) return lds ? feather::kLds256x192 : feather::kTile256x128;
    if (bm == 128 && bn == 384) return lds ? feather::kLds128x384 : feather::kTile128x128;
    if (bm >= 256 && bn >= 256) {
        if (!lds) return feather::kTile256x256;
        return feather::kLds256x256;
    }
    if (bm >= 256) return lds ? feather::kLds256x128 : feather::kTile256x128;
    if (bn >= 256) return bm >= 128 ? (lds ? feather::kLds128x256 : feather::kTile128x256) : feather::kTile64x128;
    if (bm >= 128 && bn >= 128) return lds ? feather::kLds128x128 : feather::kTile128x128;
    if (bn >= 128) return feather::kTile64x128;
    return feather::kTile64x64;
}

// Shape limits every kernel family relies on: the LDS kernels build per-lane copy offsets
// within a tile as 32-bit products (row * K * 2 over 256 rows, (3 * N + column) * 16 over a
// 4-group stage), so K < 2^22 and N < 2^25 keep them below 2^31; M and (K/16) * N stay 32-bit.
constexpr int64_t kMaxK = int64_t{1} << 22;
constexpr int64_t kMaxN = int64_t{1} << 25;

bool sizes_ok(int64_t M, int64_t N, int64_t K) {
    const int64_t lim = INT32_MAX;
    return M >= 0 && N > 0 && K > 0 && M <= lim && N < kMaxN && K < kMaxK && N % 16 == 0 && K % 16 == 0 &&
           (K / 16) * N <= lim;
}

// FEATHEROPS_GROUP_M: tile-raster group height of the tile kernels (tuning knob, default 4).
int tuning_group_m() {
    static const int g = [] {
        const char* e = getenv("FEATHEROPS_GROUP_M");
        const int v = e ? atoi(e) : 4;
        return v > 0 ? v : 4;
    }();
    return g;
}

// FEATHEROPS_SMALLM_GROUPS: workgroup count the small-M K split aims for, and the most the
// split-K LDS tiles' grid may have (tuning knob, default 256).
int tuning_smallm_groups() {
    static const int g = [] {
        const char* e = getenv("FEATHEROPS_SMALLM_GROUPS");
        const int v = e ? atoi(e) : 256;
        return v > 0 ? v : 256;
    }();
    return g;
}

// Split-K LDS tiles (64 x 64, or 32 x 128 for M <= 32) with at most 256
// workgroups, for K % 64 == 0 and
//   * 16 < M <= 32 and a weight larger than 4096 x 4096, unless the small-M
//     plan runs unsplit in one round of 16-column strips (N <= 4096): M=32
//     N=13824 K=5120 16.5 us vs 20.3 us for the small-M kernel, M=24 N=K=5120
//     10.4 vs 11.4 us, M=32 N=3072 K=12288 13.7 vs 16.6 us, but M=24 N=3280
//     K=6016 (unsplit, 205 strips) 6.9 us on the small-M kernel vs 10.2; at
//     N=K=4096 the small-M kernel wins, 6.5 vs 9.1 us at M=32, and at M <= 16
//     it wins or ties: M=16 N=13824 K=5120 15.6 vs 15.2 us, N=K=8192 15.9 vs
//     16.6 us);
//   * 32 < M <= 64: M > 48, N >= 3072, or a weight of at least 4096 x 4096
//     (the small-M kernel re-reads the activations once per 16-32 columns,
//     which past 32 rows costs more than shared LDS stages plus the split-K
//     reduction: M=64 N=13824 K=5120 20.8 us vs 83 us, M=33 N=K=3072 7.7 vs
//     11.3 us, M=40 N=8192 K=1024 5.4 vs 9.4 us, M=48 N=5120 K=3072 8.2 vs
//     15.0 us; narrower weights need 8-16 K splits and stay on the small-M
//     kernel: M=33 N=K=2048 7.1 vs 7.8 us, M=40 N=1024 K=8192 10.9 vs 11.8 us);
//   * M > 64 when the split-K plan's grid fits one round of `target`
//     workgroups (each holds a CU's LDS, so a larger grid runs twice):
//     M=154 N=10240 K=4096 19.9 us vs 32.0 us on 128 x 128 tiles, M=512
//     N=3072 K=12288 47 vs 85 us, M=1024 N=2048 K=8192 36 vs 54 us, M=2048
//     N=K=1024 7.4 vs 10.8 us; past it the tile kernel wins (M=256 N=10240
//     K=4096: 320 workgroups, 38.2 vs 32.7 us; M=768 N=K=3072 27.4 vs 22.5 us,
//     M=512 N=K=5120 44.8 vs 39.0 us, M=256 N=13824 K=5120 49.3 vs 41.2 us).
// Measured on MI355X with the C++ bench. FEATHEROPS_SPLITK (tuning knob, read
// on every call so that tests can reach the tuple's tile kernels at small
// shapes): 0 = never, 1 = always (K % 64 == 0).
int splitk_route(int64_t M, int64_t N, int64_t K) {
    const char* e = getenv("FEATHEROPS_SPLITK");
    const int v = e ? atoi(e) : -1;
    if (K % 64 != 0 || v == 0) return feather::kKernelNone;
    bool use = v == 1;
    if (!use && M <= 64)
        use = M > 48 || (M > 32 && (N >= 3072 || N * K >= int64_t(4096) * 4096)) ||
              (M > 16 && N * K > int64_t(4096) * 4096 &&
               (N > 4096 || feather::smallm_ksplit(M, N, K, tuning_smallm_groups()) > 1));
    const feather::SplitKPlan pl = feather::lds_splitk_plan(M, N, K, tuning_smallm_groups());
    if (!use && M > 64) use = static_cast<int64_t>(pl.tiles) * pl.ksplit <= tuning_smallm_groups();
    return use ? pl.kernel_id : feather::kKernelNone;
}

int kernel_for(int64_t M, int64_t N, int64_t K, int wm, int wn, int rm, int rn) {
    const int sk = splitk_route(M, N, K);
    return sk != feather::kKernelNone ? sk : tile_kernel_for(M, K, wm, wn, rm, rn);
}

bool is_splitk(int kid) {
    return kid == feather::kLdsSk64x64 || kid == feather::kLdsSk64x128 || kid == feather::kLdsSk32x128;
}

// Compute units of the current device (256 on an MI355X), read once per device.
int device_cus() {
    constexpr int kMaxDevices = 64;
    static int cus[kMaxDevices] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
    }
    return cus[dev];
}

int launch_status() { return hipGetLastError() == hipSuccess ? FEATHER_OK : FEATHER_ERR_LAUNCH; }

// ---- allocation-free K-split scratch (feather_launch_scaled_mm_noalloc) ----
// One static device array per GPU holds what a caller workspace holds for the
// K split: the 64 KB arrival-counter region, then fp32 partial tiles. The
// loader zero-fills it; every call leaves the counters at zero again. In host
// code `scratch` names a host-side stand-in, never the device memory: its
// device address comes from hipGetSymbolAddress, once per device.
constexpr size_t kNoallocScratchBytes = FEATHER_NOALLOC_SCRATCH_BYTES;
static_assert(kNoallocScratchBytes > feather::kWorkspaceCounterBytes, "scratch holds the counter region");
static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

__global__ void zero_words_kernel(uint32_t* p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Device address of `scratch` on the current device; the first call on a
// device looks it up and clears the counter region (a fill kernel on `stream`,
// ordered before the call's GEMM).
int noalloc_scratch(void** out, hipStream_t stream) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return FEATHER_ERR_INVALID;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            (void)hipGetLastError();
            return FEATHER_ERR_LAUNCH;
        }
        constexpr int kWords = static_cast<int>(feather::kWorkspaceCounterBytes / 4);
        hipLaunchKernelGGL(zero_words_kernel, dim3((kWords + 255) / 256), dim3(256), 0, stream,
                           static_cast<uint32_t*>(ptr), kWords);
        if (hipGetLastError() != hipSuccess) return FEATHER_ERR_LAUNCH;
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return FEATHER_OK;
}

}  // namespace

extern "C" {

int feather_scaled_mm_kernel_id(int64_t M, int64_t N, int64_t K, int block_warps_m, int block_warps_n, int unroll_k,
                                int repeat_m, int repeat_n) {
    if (!known_config(block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n)) return feather::kKernelNone;
    if (!sizes_ok(M, N, K)) return feather::kKernelNone;
    return kernel_for(M, N, K, block_warps_m, block_warps_n, repeat_m, repeat_n);
}

size_t feather_scaled_mm_workspace_size(int64_t M, int64_t N, int64_t K, int block_warps_m, int block_warps_n,
                                        int unroll_k, int repeat_m, int repeat_n) {
    const int kid = feather_scaled_mm_kernel_id(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n);
    if (kid == feather::kKernelNone) return 0;
    if (is_splitk(kid)) return feather::lds_splitk_plan(M, N, K, tuning_smallm_groups()).workspace_bytes;
    if (kid != feather::kSmallM) return 0;
    return feather::smallm_workspace_bytes(M, N, K, tuning_smallm_groups());
}

bool feather_launch_scaled_mm_ex(const void* a, int a_dtype, const uint8_t* b_prepacked, const float* scale,
                                 const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale,
                                 int has_bias, int block_warps_m, int block_warps_n, int unroll_k, int repeat_m,
                                 int repeat_n, int b_dtype, int output_dtype, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
    const int kid = feather_scaled_mm_kernel_id(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n);
    if (kid == feather::kKernelNone) return false;
    if (a_dtype != FEATHER_DTYPE_F16 && a_dtype != FEATHER_DTYPE_BF16) return false;
    if (b_dtype != FEATHER_B_E4M3FN && b_dtype != FEATHER_B_E5M2) return false;
    if (output_dtype != 0 && output_dtype != 1) return false;
    if (M == 0) return true;
    feather::MmArgs p;
    p.a = static_cast<const uint16_t*>(a);
    p.b = b_prepacked;
    p.scale = scale;
    p.bias = bias;
    p.c = c;
    p.M = M;
    p.N = N;
    p.K = K;
    p.has_scale = has_scale ? 1 : 0;
    p.has_bias = has_bias ? 1 : 0;
    p.out_bf16 = output_dtype == 1;
    p.b_e4m3 = b_dtype == FEATHER_B_E4M3FN;
    p.a_bf16 = a_dtype == FEATHER_DTYPE_BF16;
    p.group_m = tuning_group_m();
    p.smallm_min_groups = tuning_smallm_groups();
    if (is_splitk(kid)) return feather::launch_lds_splitk(p, workspace, workspace_bytes, stream);
    if (kid == feather::kSmallM) return feather::launch_smallm_kernel(p, workspace, workspace_bytes, stream);
    if (kid >= feather::kLds256x256) return feather::launch_lds_kernel(kid, p, stream);
    return feather::launch_tile_kernel(kid, p, stream);
}

bool feather_launch_scaled_mm_lora(const void* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                                   uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias,
                                   const uint16_t* lora_t, const uint16_t* lora_u, int64_t rank, int lora_dtype,
                                   int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n,
                                   int b_dtype, int output_dtype, hipStream_t stream) {
    const int kid = feather_scaled_mm_kernel_id(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n);
    // the rank-R epilogue exists on the large LDS tiles (fp16 activations, e5m2 weights)
    if (kid < feather::kLds256x256 || is_splitk(kid)) return false;
    if (b_dtype != FEATHER_B_E5M2 || (output_dtype != 0 && output_dtype != 1)) return false;
    if (lora_dtype != FEATHER_DTYPE_F16 && lora_dtype != FEATHER_DTYPE_BF16) return false;
    if (lora_t == nullptr || lora_u == nullptr || rank <= 0 || rank % 32 != 0 || rank > INT32_MAX / 2) return false;
    if ((reinterpret_cast<uintptr_t>(lora_t) | reinterpret_cast<uintptr_t>(lora_u)) % 16 != 0) return false;
    // the factor copies address T and U with 32-bit lane offsets
    if (M * rank * 2 > INT32_MAX || N * rank * 2 > INT32_MAX) return false;
    if (M == 0) return true;
    feather::MmArgs p;
    p.a = static_cast<const uint16_t*>(a);
    p.b = b_prepacked;
    p.scale = scale;
    p.bias = bias;
    p.c = c;
    p.M = M;
    p.N = N;
    p.K = K;
    p.has_scale = has_scale ? 1 : 0;
    p.has_bias = has_bias ? 1 : 0;
    p.out_bf16 = output_dtype == 1;
    p.b_e4m3 = false;
    p.a_bf16 = false;
    p.group_m = tuning_group_m();
    p.smallm_min_groups = tuning_smallm_groups();
    p.lora_t = lora_t;
    p.lora_u = lora_u;
    p.lora_rank = rank;
    p.lora_dtype = lora_dtype == FEATHER_DTYPE_F16 ? 1 : 2;
    return feather::launch_lds_kernel(kid, p, stream);
}

bool feather_launch_scaled_mm_ws(const void* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias,
                                 uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale, int has_bias,
                                 int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n,
                                 int b_dtype, int output_dtype, void* workspace, size_t workspace_bytes,
                                 hipStream_t stream) {
    return feather_launch_scaled_mm_ex(a, FEATHER_DTYPE_F16, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias,
                                       block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, b_dtype,
                                       output_dtype, workspace, workspace_bytes, stream);
}

int feather_launch_scaled_mm_noalloc(const void* a, int a_dtype, const uint8_t* b_prepacked, const float* scale,
                                     const uint16_t* bias, uint16_t* c, int64_t M, int64_t N, int64_t K, int has_scale,
                                     int has_bias, int block_warps_m, int block_warps_n, int unroll_k, int repeat_m,
                                     int repeat_n, int b_dtype, int output_dtype, hipStream_t stream) {
    const int kid = feather_scaled_mm_kernel_id(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n);
    if (kid == feather::kKernelNone) return FEATHER_ERR_UNSUPPORTED;
    const size_t need =
        feather_scaled_mm_workspace_size(M, N, K, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n);
    if (need > kNoallocScratchBytes) return FEATHER_ERR_SCRATCH;
    void* ws = nullptr;
    if (need > 0 && M > 0) {
        const int st = noalloc_scratch(&ws, stream);
        if (st != FEATHER_OK) return st;
    }
    if (!feather_launch_scaled_mm_ex(a, a_dtype, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias,
                                     block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, b_dtype,
                                     output_dtype, ws, ws ? kNoallocScratchBytes : 0, stream))
        return FEATHER_ERR_UNSUPPORTED;
    return launch_status();
}

bool launch_scaled_mm(const void* a, const uint8_t* b_prepacked, const float* scale, const uint16_t* bias, uint16_t* c,
                      int64_t M, int64_t N, int64_t K, int has_scale, int has_bias, int block_warps_m,
                      int block_warps_n, int unroll_k, int repeat_m, int repeat_n, int b_dtype, int output_dtype,
                      hipStream_t stream) {
    return feather_launch_scaled_mm_ws(a, b_prepacked, scale, bias, c, M, N, K, has_scale, has_bias, block_warps_m,
                                       block_warps_n, unroll_k, repeat_m, repeat_n, b_dtype, output_dtype, nullptr, 0,
                                       stream);
}

int feather_quantize_prepack_e5m2(const void* w, int w_dtype, int64_t N, int64_t K, const float* ckpt_scale,
                                  int native, uint8_t* out, float* scale_out, uint32_t* workspace, hipStream_t stream) {
    if (!w || !out || !scale_out || !workspace) return FEATHER_ERR_INVALID;
    if (w_dtype != FEATHER_DTYPE_F16 && w_dtype != FEATHER_DTYPE_BF16 && w_dtype != FEATHER_DTYPE_F32)
        return FEATHER_ERR_INVALID;
    if (N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K > INT32_MAX || (N + 63) / 64 > 65535)
        return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u)) return FEATHER_ERR_INVALID;
    feather::QuantArgs q;
    q.w = w;
    q.dtype = w_dtype;
    q.N = N;
    q.K = K;
    q.ckpt_scale = ckpt_scale;
    q.native = native != 0;
    q.out = out;
    q.scale_out = scale_out;
    q.workspace = workspace;
    q.scale_in = nullptr;
    feather::launch_quantize_prepack(q, stream);
    return launch_status();
}

size_t feather_quantize_workspace_size(void) { return feather::kWorkspaceCounterBytes + 4096; }

int feather_quantize_prepack_e5m2_ws(const void* w, int w_dtype, int64_t N, int64_t K, const float* ckpt_scale,
                                     int native, uint8_t* out, float* scale_out, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream) {
    if (!workspace || workspace_bytes < feather_quantize_workspace_size()) return FEATHER_ERR_INVALID;
    if (!w || !out || !scale_out) return FEATHER_ERR_INVALID;
    if (w_dtype != FEATHER_DTYPE_F16 && w_dtype != FEATHER_DTYPE_BF16 && w_dtype != FEATHER_DTYPE_F32)
        return FEATHER_ERR_INVALID;
    if (N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K > INT32_MAX || (N + 63) / 64 > 65535)
        return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u)) return FEATHER_ERR_INVALID;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    feather::QuantArgs q;
    q.w = w;
    q.dtype = w_dtype;
    q.N = N;
    q.K = K;
    q.ckpt_scale = ckpt_scale;
    q.native = native != 0;
    q.out = out;
    q.scale_out = scale_out;
    q.workspace = reinterpret_cast<uint32_t*>(ws + feather::kWorkspaceCounterBytes);  // partial maxima
    q.scale_in = nullptr;
    q.counters = reinterpret_cast<uint32_t*>(ws);  // two words of the zero region
    q.cus = device_cus() <= 1024 ? device_cus() : 0;
    feather::launch_quantize_prepack(q, stream);
    return launch_status();
}

int feather_quantize_prepack_e5m2_scaled(const void* w, int w_dtype, int64_t N, int64_t K, const float* scale,
                                         uint8_t* out, hipStream_t stream) {
    if (!w || !out || !scale) return FEATHER_ERR_INVALID;
    if (w_dtype != FEATHER_DTYPE_F16 && w_dtype != FEATHER_DTYPE_BF16 && w_dtype != FEATHER_DTYPE_F32)
        return FEATHER_ERR_INVALID;
    if (N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K > INT32_MAX || (N + 63) / 64 > 65535)
        return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(w) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u)) return FEATHER_ERR_INVALID;
    feather::QuantArgs q;
    q.w = w;
    q.dtype = w_dtype;
    q.N = N;
    q.K = K;
    q.ckpt_scale = nullptr;
    q.native = true;
    q.out = out;
    q.scale_out = nullptr;
    q.workspace = nullptr;
    q.scale_in = scale;
    feather::launch_quantize_prepack(q, stream);
    return launch_status();
}

int feather_prepack_transpose(const uint8_t* w_nk, uint8_t* out, int64_t N, int64_t K, hipStream_t stream) {
    if (!w_nk || !out || N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K > INT32_MAX || (N + 63) / 64 > 65535)
        return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(w_nk) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u))
        return FEATHER_ERR_INVALID;
    feather::launch_chunk_transpose(w_nk, out, N, K, 0, stream);
    return launch_status();
}

int feather_unprepack_transpose(const uint8_t* packed, uint8_t* out_nk, int64_t N, int64_t K, hipStream_t stream) {
    if (!packed || !out_nk || N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K > INT32_MAX ||
        (N + 63) / 64 > 65535)
        return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(packed) & 15u) || (reinterpret_cast<uintptr_t>(out_nk) & 15u))
        return FEATHER_ERR_INVALID;
    feather::launch_chunk_transpose(packed, out_nk, N, K, 1, stream);
    return launch_status();
}

int feather_prepack_b(const uint8_t* b_kn, uint8_t* out, int64_t K, int64_t N, hipStream_t stream) {
    if (!b_kn || !out || N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K / 16 > 65535 ||
        K * N > INT64_C(1) << 40)
        return FEATHER_ERR_INVALID;
    if (reinterpret_cast<uintptr_t>(out) & 15u) return FEATHER_ERR_INVALID;
    feather::launch_prepack_kn(b_kn, out, K, N, stream);
    return launch_status();
}

int feather_bf16_to_fp16(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream) {
    if (n < 0 || (n > 0 && (!in || !out))) return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(in) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u)) return FEATHER_ERR_INVALID;
    if (n == 0) return FEATHER_OK;
    feather::launch_bf16_to_fp16(in, out, n, false, stream);
    return launch_status();
}

int feather_bf16_to_fp16_rne(const uint16_t* in, uint16_t* out, int64_t n, hipStream_t stream) {
    if (n < 0 || (n > 0 && (!in || !out))) return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(in) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u)) return FEATHER_ERR_INVALID;
    if (n == 0) return FEATHER_OK;
    feather::launch_bf16_to_fp16(in, out, n, true, stream);
    return launch_status();
}

int feather_dequantize_e5m2(const uint8_t* packed, const float* scale, void* out, int out_dtype, int64_t N, int64_t K,
                            hipStream_t stream) {
    if (!packed || !scale || !out || N <= 0 || K <= 0 || K % 16 != 0 || N > INT32_MAX || K > INT32_MAX ||
        (N + 63) / 64 > 65535)
        return FEATHER_ERR_INVALID;
    if (out_dtype != FEATHER_DTYPE_F16 && out_dtype != FEATHER_DTYPE_BF16 && out_dtype != FEATHER_DTYPE_F32)
        return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(packed) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u))
        return FEATHER_ERR_INVALID;
    feather::launch_dequant(packed, scale, out, N, K, out_dtype, stream);
    return launch_status();
}

size_t feather_lora_down_workspace_size(int64_t M, int64_t K, int64_t R) {
    if (M <= 0 || K <= 0 || R <= 0 || R % 32 != 0) return 0;
    return feather::lora_down_workspace_bytes(M, K, R);
}

int feather_lora_down(const void* x, int x_dtype, const void* d, void* t, int64_t M, int64_t K, int64_t R,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (x_dtype != FEATHER_DTYPE_F16 && x_dtype != FEATHER_DTYPE_BF16) return FEATHER_ERR_INVALID;
    if (M < 0 || K <= 0 || R <= 0 || M > INT32_MAX || R > 65536) return FEATHER_ERR_INVALID;
    // per-lane copy offsets within a tile (up to 128 rows of D) are 32-bit: 128 * K * 2 < 2^32
    if (K % 8 != 0 || R % 32 != 0 || K >= (int64_t{1} << 24)) return FEATHER_ERR_UNSUPPORTED;
    if (M == 0) return FEATHER_OK;
    if (!x || !d || !t) return FEATHER_ERR_INVALID;
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(d) | reinterpret_cast<uintptr_t>(t)) % 16 != 0)
        return FEATHER_ERR_INVALID;
    feather::LoraDownArgs a;
    a.x = static_cast<const uint16_t*>(x);
    a.d = static_cast<const uint16_t*>(d);
    a.t = static_cast<uint16_t*>(t);
    a.M = M;
    a.K = K;
    a.R = R;
    a.bf16 = x_dtype == FEATHER_DTYPE_BF16;
    feather::launch_lora_down(a, workspace, workspace_bytes, stream);
    return launch_status();
}

const char* feather_status_string(int status) {
    switch (status) {
        case FEATHER_OK: return "ok";
        case FEATHER_ERR_INVALID: return "invalid argument";
        case FEATHER_ERR_UNSUPPORTED: return "unsupported configuration";
        case FEATHER_ERR_LAUNCH: return "kernel launch failed";
        case FEATHER_ERR_SCRATCH: return "call needs more K-split scratch than the static array holds";
        default: return "unknown status";
    }
}

int feather_scaled_mm_pick_config(int64_t M, int64_t N, int64_t K, int* cfg) {
    if (!cfg || M < 0 || !sizes_ok(M, N, K)) return FEATHER_ERR_INVALID;
    // Output tiles, their measured throughput per CU relative to 256 x 256
    // (M=32768, N=13824, K=5120 and M=4096, N=3072, K=3072 on MI355X), and the
    // tuple that selects them. Cost of a tile = waves of workgroups x tile
    // area / relative throughput; shapes too small for any of them are routed
    // to the split-K tiles by the dispatcher whatever the tuple.
    struct Cand {
        Cfg c;
        int bm, bn;
        double eff;
    };
    static const Cand cands[] = {
        {{2, 4, 4, 8, 4}, 256, 256, 1.00}, {{2, 4, 4, 8, 3}, 256, 192, 0.85}, {{2, 4, 4, 4, 4}, 128, 256, 0.90},
        {{4, 2, 4, 4, 4}, 256, 128, 0.84}, {{2, 2, 4, 4, 4}, 128, 128, 0.80}, {{2, 4, 4, 4, 6}, 128, 384, 0.87},
    };
    Cfg best = {1, 1, 2, 1, 2};  // M <= 64: the small-M kernel
    if (M > 64) {
        const int cus = device_cus();
        double best_cost = 0.0;
        bool have = false;
        for (const Cand& c : cands) {
            const int64_t tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
            const double cost = static_cast<double>((tiles + cus - 1) / cus) * c.bm * c.bn / c.eff;
            if (!have || cost < best_cost) {
                best = c.c;
                best_cost = cost;
                have = true;
            }
        }
    }
    cfg[0] = best.wm;
    cfg[1] = best.wn;
    cfg[2] = best.u;
    cfg[3] = best.rm;
    cfg[4] = best.rn;
    return FEATHER_OK;
}

int feather_abi_version(void) { return 1; }

}  // extern "C"
