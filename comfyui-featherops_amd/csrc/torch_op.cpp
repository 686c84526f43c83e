// torch ops of the library, registered in C++ so that an eager call goes from
// torch's dispatcher straight to the launch entry without a Python frame:
//   feather_ops::scaled_mm        the reference's op (kernel/hip/hip_kernel.cu:
//                                 746-767: same namespace, schema, CUDA key)
//   feather_ops::scaled_mm_any_m  any M, shape-picked tile, fp16/bf16 A (no
//                                 counterpart in the reference; Meta kernel for
//                                 fake tensors)
//   feather_ops::scaled_mm_any_m_lora
//                                 the any-M op plus an unmerged-LoRA term,
//                                 fused into the epilogue on the large tiles
//   feather_ops::quantize_prepack_e5m2(_scaled)
//                                 the fused quantize + prepack of a weight
//   feather_ops::lora_down        T = F.linear(x, d), the LoRA down-projection
//                                 of all patches at once
//   feather_ops_internal::scaled_mm_configured
//                                 the reference's configured op (hip_kernel.py:
//                                 12-58, a Python custom op there), Meta kernel
//
// Checks and messages follow the reference's scaled_mm (hip_kernel.cu:648-730);
// the stride of a dimension of size 1 is never read, so any value passes.
// Launches go to torch's current HIP stream of a's device. The K-split kernels
// get a per-(device, stream) workspace: zero-filled when first allocated, and
// left with its counter region zero by every call, whatever the shape.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <utility>

#include "featherops_amd.h"

namespace {

at::Tensor& workspace_for(const at::Device& dev, hipStream_t stream, size_t nbytes) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, at::Tensor> pool;
    std::lock_guard<std::mutex> lock(mu);
    at::Tensor& ws = pool[{dev.index(), stream}];
    if (!ws.defined() || static_cast<size_t>(ws.numel()) < nbytes) {
        const int64_t n = static_cast<int64_t>(nbytes > (size_t(1) << 20) ? nbytes : (size_t(1) << 20));
        ws = at::zeros({n}, at::TensorOptions().dtype(at::kByte).device(dev));
    }
    return ws;
}

// Argument checks of the reference's scaled_mm (hip_kernel.cu:648-730).
// `block_divisible = false` replaces the BlockM/BlockN/ChunkK divisibility
// rules by what the gfx950 kernels need (N % 16 == 0; K % 16 is always
// required) and `allow_bf16_a` accepts bf16 activations: the any-M entry.
void check_args(const at::Tensor& a, const at::Tensor& b_prepacked, const std::optional<at::Tensor>& scale,
                const std::optional<at::Tensor>& bias, const at::Tensor& c, int64_t block_warps_m,
                int64_t block_warps_n, int64_t unroll_k, int64_t repeat_m, int64_t repeat_n, int64_t b_dtype,
                bool block_divisible, bool allow_bf16_a) {
    TORCH_CHECK(a.is_cuda(), "a must be a CUDA tensor");
    TORCH_CHECK(b_prepacked.is_cuda(), "b_prepacked must be a CUDA tensor");
    TORCH_CHECK(c.is_cuda(), "c must be a CUDA tensor");
    TORCH_CHECK(b_prepacked.device() == a.device(), "b_prepacked must be on the same device as a");
    TORCH_CHECK(c.device() == a.device(), "c must be on the same device as a");
    if (allow_bf16_a) {
        TORCH_CHECK(a.scalar_type() == at::kHalf || a.scalar_type() == at::kBFloat16, "a must be float16 or bfloat16");
    } else {
        TORCH_CHECK(a.scalar_type() == at::kHalf, "a must be float16");
    }
    TORCH_CHECK(c.scalar_type() == at::kHalf || c.scalar_type() == at::kBFloat16, "c must be float16 or bfloat16");
    TORCH_CHECK(b_dtype == 0 || b_dtype == 1, "b_dtype must be 0 (fp8e4m3) or 1 (fp8e5m2)");
    if (b_dtype == 0) {
        TORCH_CHECK(b_prepacked.scalar_type() == at::kFloat8_e4m3fn, "b_prepacked must be float8_e4m3fn when b_dtype=0");
    } else {
        TORCH_CHECK(b_prepacked.scalar_type() == at::kFloat8_e5m2, "b_prepacked must be float8_e5m2 when b_dtype=1");
    }
    TORCH_CHECK(a.dim() == 2, "a must be 2D");
    TORCH_CHECK(b_prepacked.dim() == 3, "b_prepacked must be 3D (K/16, N, 16)");
    TORCH_CHECK(c.dim() == 2, "c must be 2D");
    const int64_t M = a.size(0), K = a.size(1), N = b_prepacked.size(1);
    TORCH_CHECK(K % 16 == 0, "K must be divisible by 16");
    TORCH_CHECK(b_prepacked.size(0) == K / 16, "b_prepacked.shape[0] must equal K/16 (", K / 16, ")");
    TORCH_CHECK(b_prepacked.size(2) == 16, "b_prepacked.shape[2] must be 16");
    TORCH_CHECK(c.size(0) == M, "c.shape[0] must equal M");
    TORCH_CHECK(c.size(1) == N, "c.shape[1] must equal N");
    TORCH_CHECK(M == 1 || a.stride(0) == K, "a.stride(0) must equal K (", K, ")");
    TORCH_CHECK(a.stride(1) == 1, "a.stride(1) must be 1");
    TORCH_CHECK(K / 16 == 1 || b_prepacked.stride(0) == N * 16, "b_prepacked.stride(0) must equal N*16 (", N * 16, ")");
    TORCH_CHECK(b_prepacked.stride(1) == 16, "b_prepacked.stride(1) must be 16");
    TORCH_CHECK(b_prepacked.stride(2) == 1, "b_prepacked.stride(2) must be 1");
    TORCH_CHECK(M == 1 || c.stride(0) == N, "c.stride(0) must equal N (", N, ")");
    TORCH_CHECK(c.stride(1) == 1, "c.stride(1) must be 1");
    if (scale.has_value()) {
        TORCH_CHECK(scale->is_cuda(), "scale must be a CUDA tensor");
        TORCH_CHECK(scale->device() == a.device(), "scale must be on the same device as a");
        TORCH_CHECK(scale->scalar_type() == at::kFloat, "scale must be float32");
        TORCH_CHECK(scale->numel() == 1, "scale must have one element");
    }
    if (bias.has_value()) {
        TORCH_CHECK(bias->is_cuda(), "bias must be a CUDA tensor");
        TORCH_CHECK(bias->device() == a.device(), "bias must be on the same device as a");
        TORCH_CHECK(bias->scalar_type() == c.scalar_type(), "bias must have the same dtype as c");
        TORCH_CHECK(bias->numel() == N, "bias must have N elements");
    }
    TORCH_CHECK(reinterpret_cast<uintptr_t>(a.data_ptr()) % 16 == 0, "a data pointer must be 16-byte aligned");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(b_prepacked.data_ptr()) % 16 == 0,
                "b_prepacked data pointer must be 16-byte aligned");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(c.data_ptr()) % 16 == 0, "c data pointer must be 16-byte aligned");
    const int64_t block_m = 16 * block_warps_m * repeat_m;
    const int64_t block_n = 16 * block_warps_n * repeat_n;
    const int64_t chunk_k = 16 * unroll_k;
    if (block_divisible) {
        TORCH_CHECK(block_m > 0 && M % block_m == 0, "M (", M, ") must be divisible by kBlockM (", block_m, ")");
        TORCH_CHECK(block_n > 0 && N % block_n == 0, "N (", N, ") must be divisible by kBlockN (", block_n, ")");
        TORCH_CHECK(chunk_k > 0 && K % chunk_k == 0, "K (", K, ") must be divisible by kChunkK (", chunk_k, ")");
    } else {
        TORCH_CHECK(N % 16 == 0, "N (", N, ") must be divisible by 16");
    }
    TORCH_CHECK(32 * block_warps_m * block_warps_n <= 1024, "Block size exceeds HIP thread-per-block limit");
}

struct Launch {
    const at::Tensor& b_prepacked;
    const std::optional<at::Tensor>& scale;
    const std::optional<at::Tensor>& bias;
    const at::Tensor& c;
    int64_t M, N, K;
    int cfg[5];
    int b_dtype;
    void* ws;
    size_t ws_size;
    hipStream_t stream;

    bool operator()(const at::Tensor& a, int a_dtype) const {
        return feather_launch_scaled_mm_ex(
            a.data_ptr(), a_dtype, static_cast<const uint8_t*>(b_prepacked.data_ptr()),
            scale.has_value() ? static_cast<const float*>(scale->data_ptr()) : nullptr,
            bias.has_value() ? static_cast<const uint16_t*>(bias->data_ptr()) : nullptr,
            static_cast<uint16_t*>(c.data_ptr()), M, N, K, scale.has_value() ? 1 : 0, bias.has_value() ? 1 : 0,
            cfg[0], cfg[1], cfg[2], cfg[3], cfg[4], b_dtype, c.scalar_type() == at::kHalf ? 0 : 1, ws, ws_size,
            stream);
    }
};

// Enqueue the GEMM for config `cfg` on torch's current stream of a's device
// (the caller holds a device guard for it).
Launch make_launch(const at::Tensor& a, const at::Tensor& b_prepacked, const std::optional<at::Tensor>& scale,
                   const std::optional<at::Tensor>& bias, const at::Tensor& c, const int (&cfg)[5], int b_dtype) {
    const hipStream_t stream = c10::hip::getCurrentHIPStream(a.device().index()).stream();
    const int64_t M = a.size(0), K = a.size(1), N = b_prepacked.size(1);
    Launch l{b_prepacked, scale, bias, c, M, N, K, {cfg[0], cfg[1], cfg[2], cfg[3], cfg[4]}, b_dtype, nullptr, 0,
             stream};
    const size_t ws_bytes = feather_scaled_mm_workspace_size(M, N, K, cfg[0], cfg[1], cfg[2], cfg[3], cfg[4]);
    if (ws_bytes) {
        at::Tensor& t = workspace_for(a.device(), stream, ws_bytes);
        l.ws = t.data_ptr();
        l.ws_size = static_cast<size_t>(t.numel());
    }
    return l;
}

// feather_ops::scaled_mm (hip_kernel.cu:648-743): writes c for the given config.
void scaled_mm(const at::Tensor& a, const at::Tensor& b_prepacked, const std::optional<at::Tensor>& scale,
               const std::optional<at::Tensor>& bias, const at::Tensor& c, int64_t block_warps_m,
               int64_t block_warps_n, int64_t unroll_k, int64_t repeat_m, int64_t repeat_n, int64_t b_dtype) {
    check_args(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n, b_dtype,
               true, false);
    const c10::DeviceGuard guard(a.device());
    const int cfg[5] = {static_cast<int>(block_warps_m), static_cast<int>(block_warps_n), static_cast<int>(unroll_k),
                        static_cast<int>(repeat_m), static_cast<int>(repeat_n)};
    TORCH_CHECK(make_launch(a, b_prepacked, scale, bias, c, cfg, static_cast<int>(b_dtype))(a, FEATHER_DTYPE_F16),
                "Unsupported config");
}

// feather_ops::scaled_mm_any_m: any row count M without padding (the kernels
// mask rows past M), the tile from feather_scaled_mm_pick_config, fp16 or bf16
// activations. bf16 activations are rounded to fp16 inside the small-M kernel,
// otherwise by the library's round-to-nearest-even cast first: the values of
// x.to(float16) (comfy_feather/ops.py:88) either way.
at::Tensor scaled_mm_any_m(const at::Tensor& a, const at::Tensor& b_prepacked, const std::optional<at::Tensor>& scale,
                           const std::optional<at::Tensor>& bias, at::ScalarType out_dtype) {
    TORCH_CHECK(a.dim() == 2, "a must be 2D");
    TORCH_CHECK(b_prepacked.dim() == 3, "b_prepacked must be 3D (K/16, N, 16)");
    const int64_t M = a.size(0), K = a.size(1), N = b_prepacked.size(1);
    at::Tensor c = at::empty({M, N}, a.options().dtype(out_dtype));
    if (M == 0) return c;
    const c10::DeviceGuard guard(a.device());
    int cfg[5];
    const int status = feather_scaled_mm_pick_config(M, N, K, cfg);
    TORCH_CHECK(status == FEATHER_OK, "feather_scaled_mm_pick_config failed: ", feather_status_string(status));
    const int b_dtype = b_prepacked.scalar_type() == at::kFloat8_e4m3fn ? 0 : 1;
    check_args(a, b_prepacked, scale, bias, c, cfg[0], cfg[1], cfg[2], cfg[3], cfg[4], b_dtype, false, true);
    const Launch launch = make_launch(a, b_prepacked, scale, bias, c, cfg, b_dtype);
    bool launched;
    if (a.scalar_type() == at::kBFloat16) {
        launched = launch(a, FEATHER_DTYPE_BF16);
        if (!launched) {
            const at::Tensor a16 = at::empty(a.sizes(), a.options().dtype(at::kHalf));
            const int st = feather_bf16_to_fp16_rne(static_cast<const uint16_t*>(a.data_ptr()),
                                                   static_cast<uint16_t*>(a16.data_ptr()), a.numel(), launch.stream);
            TORCH_CHECK(st == FEATHER_OK, "feather_bf16_to_fp16_rne failed: ", feather_status_string(st));
            launched = launch(a16, FEATHER_DTYPE_F16);
        }
    } else {
        launched = launch(a, FEATHER_DTYPE_F16);
    }
    TORCH_CHECK(launched, "Unsupported config");
    return c;
}

// feather_ops_internal::scaled_mm_configured (reference kernel/hip/hip_kernel.py:
// 12-39): allocates C (M, N) of out_dtype and runs feather_ops::scaled_mm with
// the weight dtype's code (e4m3fn -> 0, otherwise 1).
at::Tensor scaled_mm_configured(const at::Tensor& a, const at::Tensor& b_prepacked,
                                const std::optional<at::Tensor>& scale, const std::optional<at::Tensor>& bias,
                                at::ScalarType out_dtype, int64_t block_warps_m, int64_t block_warps_n,
                                int64_t unroll_k, int64_t repeat_m, int64_t repeat_n) {
    TORCH_CHECK(a.dim() == 2, "a must be 2D");
    TORCH_CHECK(b_prepacked.dim() == 3, "b_prepacked must be 3D (K/16, N, 16)");
    at::Tensor c = at::empty({a.size(0), b_prepacked.size(1)}, a.options().dtype(out_dtype));
    scaled_mm(a, b_prepacked, scale, bias, c, block_warps_m, block_warps_n, unroll_k, repeat_m, repeat_n,
              b_prepacked.scalar_type() == at::kFloat8_e4m3fn ? 0 : 1);
    return c;
}

at::Tensor scaled_mm_configured_meta(const at::Tensor& a, const at::Tensor& b_prepacked,
                                     const std::optional<at::Tensor>& scale, const std::optional<at::Tensor>& bias,
                                     at::ScalarType out_dtype, int64_t, int64_t, int64_t, int64_t, int64_t) {
    return at::empty({a.size(0), b_prepacked.size(1)}, a.options().dtype(out_dtype));
}

// feather_ops::scaled_mm_any_m_lora: scaled_mm_any_m plus the unmerged-LoRA
// term T . U^T (reference comfy_feather/lora.py:4-35, after F.linear(x, A);
// the strengths are folded into T by the caller). T (M, R) and U (N, R) are
// contiguous fp16 or bf16 with R % 32 == 0. On the large LDS tiles the term is
// added to the scaled fp32 accumulator before rounding; on every other route
// the GEMM runs as scaled_mm_any_m and the term is added to C afterwards.
at::Tensor scaled_mm_any_m_lora(const at::Tensor& a, const at::Tensor& b_prepacked,
                                const std::optional<at::Tensor>& scale, const std::optional<at::Tensor>& bias,
                                at::ScalarType out_dtype, const at::Tensor& lora_t, const at::Tensor& lora_u) {
    TORCH_CHECK(a.dim() == 2, "a must be 2D");
    TORCH_CHECK(b_prepacked.dim() == 3, "b_prepacked must be 3D (K/16, N, 16)");
    const int64_t M = a.size(0), K = a.size(1), N = b_prepacked.size(1);
    TORCH_CHECK(lora_t.is_cuda() && lora_u.is_cuda() && lora_t.device() == a.device() && lora_u.device() == a.device(),
                "lora_t and lora_u must be CUDA tensors on a's device");
    TORCH_CHECK(lora_t.scalar_type() == lora_u.scalar_type() &&
                    (lora_t.scalar_type() == at::kHalf || lora_t.scalar_type() == at::kBFloat16),
                "lora_t and lora_u must both be float16 or both bfloat16");
    TORCH_CHECK(lora_t.dim() == 2 && lora_u.dim() == 2 && lora_t.size(0) == M && lora_u.size(0) == N &&
                    lora_t.size(1) == lora_u.size(1),
                "lora_t must be (M, R) and lora_u (N, R)");
    const int64_t R = lora_t.size(1);
    TORCH_CHECK(R > 0 && R % 32 == 0, "lora rank must be a positive multiple of 32 (pad with zero columns)");
    TORCH_CHECK(lora_t.is_contiguous() && lora_u.is_contiguous(), "lora_t and lora_u must be contiguous");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(lora_t.data_ptr()) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(lora_u.data_ptr()) % 16 == 0,
                "lora_t and lora_u data pointers must be 16-byte aligned");
    if (M == 0) return at::empty({M, N}, a.options().dtype(out_dtype));
    const c10::DeviceGuard guard(a.device());
    int cfg[5];
    const int status = feather_scaled_mm_pick_config(M, N, K, cfg);
    TORCH_CHECK(status == FEATHER_OK, "feather_scaled_mm_pick_config failed: ", feather_status_string(status));
    const int b_dtype = b_prepacked.scalar_type() == at::kFloat8_e4m3fn ? 0 : 1;
    int kid = feather_scaled_mm_kernel_id(M, N, K, cfg[0], cfg[1], cfg[2], cfg[3], cfg[4]);
    if (kid == 26) {
        // the 128 x 384 tile's stage buffers cannot hold 64 ranks of its U rows, so it has no rank-R
        // epilogue: the 256 x 192 tile covers the same grids (256 tiles at M = 4096, N = 3072)
        const int alt[5] = {2, 4, 4, 8, 3};
        for (int i = 0; i < 5; ++i) cfg[i] = alt[i];
        kid = feather_scaled_mm_kernel_id(M, N, K, cfg[0], cfg[1], cfg[2], cfg[3], cfg[4]);
    }
    // the fused epilogue: large LDS tiles (kernel ids 20-29 but 26), e5m2 weights
    if (kid >= 20 && kid < 30 && b_dtype == 1) {
        at::Tensor c = at::empty({M, N}, a.options().dtype(out_dtype));
        check_args(a, b_prepacked, scale, bias, c, cfg[0], cfg[1], cfg[2], cfg[3], cfg[4], b_dtype, false, true);
        const hipStream_t stream = c10::hip::getCurrentHIPStream(a.device().index()).stream();
        at::Tensor a16 = a;
        if (a.scalar_type() == at::kBFloat16) {  // the large tiles take fp16 activations
            a16 = at::empty(a.sizes(), a.options().dtype(at::kHalf));
            const int st = feather_bf16_to_fp16_rne(static_cast<const uint16_t*>(a.data_ptr()),
                                                    static_cast<uint16_t*>(a16.data_ptr()), a.numel(), stream);
            TORCH_CHECK(st == FEATHER_OK, "feather_bf16_to_fp16_rne failed: ", feather_status_string(st));
        }
        const bool launched = feather_launch_scaled_mm_lora(
            a16.data_ptr(), static_cast<const uint8_t*>(b_prepacked.data_ptr()),
            scale.has_value() ? static_cast<const float*>(scale->data_ptr()) : nullptr,
            bias.has_value() ? static_cast<const uint16_t*>(bias->data_ptr()) : nullptr,
            static_cast<uint16_t*>(c.data_ptr()), M, N, K, scale.has_value() ? 1 : 0, bias.has_value() ? 1 : 0,
            static_cast<const uint16_t*>(lora_t.data_ptr()), static_cast<const uint16_t*>(lora_u.data_ptr()), R,
            lora_t.scalar_type() == at::kHalf ? FEATHER_DTYPE_F16 : FEATHER_DTYPE_BF16, cfg[0], cfg[1], cfg[2],
            cfg[3], cfg[4], b_dtype, out_dtype == at::kHalf ? 0 : 1, stream);
        if (launched) return c;
    }
    at::Tensor c = scaled_mm_any_m(a, b_prepacked, scale, bias, out_dtype);
    c.add_(at::mm(lora_t, lora_u.t()).to(out_dtype));
    return c;
}

at::Tensor scaled_mm_any_m_lora_meta(const at::Tensor& a, const at::Tensor& b_prepacked,
                                     const std::optional<at::Tensor>& scale, const std::optional<at::Tensor>& bias,
                                     at::ScalarType out_dtype, const at::Tensor& lora_t, const at::Tensor& lora_u) {
    return at::empty({a.size(0), b_prepacked.size(1)}, a.options().dtype(out_dtype));
}

// feather_ops::lora_down: T = F.linear(x, d) for the fused LoRA epilogue (the first
// F.linear of the reference's comfy_feather/lora.py:4-35, all patches stacked
// along the rank): x (M, K) and d (R, K) contiguous in the same dtype (fp16 or
// bf16), K % 8 == 0, R % 32 == 0; T (M, R) in that dtype, fp32 accumulation.
at::Tensor lora_down(const at::Tensor& x, const at::Tensor& d) {
    TORCH_CHECK(x.is_cuda() && d.is_cuda() && d.device() == x.device(), "x and d must be CUDA tensors on one device");
    TORCH_CHECK(x.dim() == 2 && d.dim() == 2 && x.size(1) == d.size(1), "x must be (M, K) and d (R, K)");
    TORCH_CHECK(x.scalar_type() == d.scalar_type() &&
                    (x.scalar_type() == at::kHalf || x.scalar_type() == at::kBFloat16),
                "x and d must both be float16 or both bfloat16");
    TORCH_CHECK(x.is_contiguous() && d.is_contiguous(), "x and d must be contiguous");
    const int64_t M = x.size(0), K = x.size(1), R = d.size(0);
    TORCH_CHECK(K % 8 == 0 && R > 0 && R % 32 == 0, "lora_down needs K % 8 == 0 and R a positive multiple of 32");
    at::Tensor t = at::empty({M, R}, x.options());
    if (M == 0) return t;
    const c10::DeviceGuard guard(x.device());
    const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    const size_t ws_bytes = feather_lora_down_workspace_size(M, K, R);
    void* ws = ws_bytes ? workspace_for(x.device(), stream, ws_bytes).data_ptr() : nullptr;
    const int st = feather_lora_down(x.data_ptr(), x.scalar_type() == at::kHalf ? FEATHER_DTYPE_F16 : FEATHER_DTYPE_BF16,
                                     d.data_ptr(), t.data_ptr(), M, K, R, ws, ws_bytes, stream);
    TORCH_CHECK(st == FEATHER_OK, "feather_lora_down failed: ", feather_status_string(st));
    return t;
}

at::Tensor lora_down_meta(const at::Tensor& x, const at::Tensor& d) {
    return at::empty({x.size(0), d.size(0)}, x.options());
}

int weight_dtype_code(const at::Tensor& w) {
    switch (w.scalar_type()) {
        case at::kHalf: return FEATHER_DTYPE_F16;
        case at::kBFloat16: return FEATHER_DTYPE_BF16;
        case at::kFloat: return FEATHER_DTYPE_F32;
        default:
            TORCH_CHECK(false, "FeatherOps quantization supports float16, bfloat16 and float32 inputs, got ",
                        w.scalar_type());
    }
    return -1;
}

void check_weight(const at::Tensor& w) {
    TORCH_CHECK(w.is_cuda(), "w must be a CUDA tensor");
    TORCH_CHECK(w.dim() == 2, "w must be 2D (N, K)");
    TORCH_CHECK(w.size(1) % 16 == 0, "K (", w.size(1), ") must be divisible by 16");
}

// feather_ops::quantize_prepack_e5m2 (reference comfy_feather/quant.py:52-74 +
// prepack_transpose, quant.py:11-13): (N, K) fp16/bf16/fp32 weight -> the
// (K/16, N, 16) e5m2 codes and the fp32 per-tensor scale. native = false is
// the load path (fp32 arithmetic on w * ckpt_scale), native = true the patch
// path (arithmetic in w's dtype, fp16 reciprocal clamp).
std::tuple<at::Tensor, at::Tensor> quantize_prepack_e5m2(const at::Tensor& w, const std::optional<at::Tensor>& ckpt_scale,
                                                         bool native) {
    check_weight(w);
    const int code = weight_dtype_code(w);
    const at::Tensor src = w.contiguous();
    const int64_t N = src.size(0), K = src.size(1);
    const c10::DeviceGuard guard(src.device());
    at::Tensor out = at::empty({K / 16, N, 16}, src.options().dtype(at::kFloat8_e5m2));
    at::Tensor scale = at::empty({}, src.options().dtype(at::kFloat));
    at::Tensor cs;
    if (ckpt_scale.has_value()) cs = ckpt_scale->reshape({1}).to(src.device(), at::kFloat).contiguous();
    const hipStream_t stream = c10::hip::getCurrentHIPStream(src.device().index()).stream();
    // the stream's zero-filled workspace (its counter region is left zero)
    const size_t ws_bytes = feather_quantize_workspace_size();
    at::Tensor& ws = workspace_for(src.device(), stream, ws_bytes);
    const int st = feather_quantize_prepack_e5m2_ws(src.data_ptr(), code, N, K,
                                                    cs.defined() ? static_cast<const float*>(cs.data_ptr()) : nullptr,
                                                    native ? 1 : 0, static_cast<uint8_t*>(out.data_ptr()),
                                                    static_cast<float*>(scale.data_ptr()), ws.data_ptr(),
                                                    static_cast<size_t>(ws.numel()), stream);
    TORCH_CHECK(st == FEATHER_OK, "quantize_prepack failed: ", feather_status_string(st), " (status ", st, ")");
    return {out, scale};
}

// feather_ops::quantize_prepack_e5m2_scaled: the same with a given scale
// (quant.py:59-74 when `scale` is passed; no amax, no clamp).
at::Tensor quantize_prepack_e5m2_scaled(const at::Tensor& w, const at::Tensor& scale) {
    check_weight(w);
    const int code = weight_dtype_code(w);
    const at::Tensor src = w.contiguous();
    const int64_t N = src.size(0), K = src.size(1);
    const c10::DeviceGuard guard(src.device());
    at::Tensor out = at::empty({K / 16, N, 16}, src.options().dtype(at::kFloat8_e5m2));
    const at::Tensor s = scale.reshape({1}).to(src.device(), at::kFloat).contiguous();
    const hipStream_t stream = c10::hip::getCurrentHIPStream(src.device().index()).stream();
    const int st = feather_quantize_prepack_e5m2_scaled(src.data_ptr(), code, N, K,
                                                        static_cast<const float*>(s.data_ptr()),
                                                        static_cast<uint8_t*>(out.data_ptr()), stream);
    TORCH_CHECK(st == FEATHER_OK, "quantize_prepack failed: ", feather_status_string(st), " (status ", st, ")");
    return out;
}

// feather_ops::bf16_to_fp16: the bf16 -> fp16 casts of kernel/convert.py,
// registered in C++ so that a call costs one dispatch (small tensors are bound
// by the host). rne = false: the reference's round-toward-zero cast
// (kernel/convert.py:24-34, saturating at +-65504; the Python entry keeps its
// even-length assertion, the kernel takes any length); rne = true: round to
// nearest even, the values of x.to(torch.float16).
at::Tensor bf16_to_fp16(const at::Tensor& x, bool rne) {
    TORCH_CHECK(x.is_cuda(), "x must be a CUDA tensor");
    TORCH_CHECK(x.scalar_type() == at::kBFloat16, "x must be bfloat16");
    TORCH_CHECK(x.is_contiguous(), "x must be contiguous");
    TORCH_CHECK(reinterpret_cast<uintptr_t>(x.data_ptr()) % 16 == 0, "x data pointer must be 16-byte aligned");
    at::Tensor out = at::empty(x.sizes(), x.options().dtype(at::kHalf));
    if (x.numel() == 0) return out;
    const c10::DeviceGuard guard(x.device());
    const hipStream_t stream = c10::hip::getCurrentHIPStream(x.device().index()).stream();
    const auto* in = static_cast<const uint16_t*>(x.data_ptr());
    auto* o = static_cast<uint16_t*>(out.data_ptr());
    const int st = rne ? feather_bf16_to_fp16_rne(in, o, x.numel(), stream) : feather_bf16_to_fp16(in, o, x.numel(), stream);
    TORCH_CHECK(st == FEATHER_OK, "bf16_to_fp16 failed: ", feather_status_string(st), " (status ", st, ")");
    return out;
}

at::Tensor bf16_to_fp16_meta(const at::Tensor& x, bool) { return at::empty(x.sizes(), x.options().dtype(at::kHalf)); }

at::Tensor scaled_mm_any_m_meta(const at::Tensor& a, const at::Tensor& b_prepacked,
                                const std::optional<at::Tensor>& scale, const std::optional<at::Tensor>& bias,
                                at::ScalarType out_dtype) {
    return at::empty({a.size(0), b_prepacked.size(1)}, a.options().dtype(out_dtype));
}

}  // namespace

TORCH_LIBRARY(feather_ops, m) {
    m.def("scaled_mm(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, Tensor(a!) c, int block_warps_m, "
          "int block_warps_n, int unroll_k, int repeat_m, int repeat_n, int b_dtype) -> ()");
    m.def("scaled_mm_any_m(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, ScalarType out_dtype) -> Tensor");
    m.def("scaled_mm_any_m_lora(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, ScalarType out_dtype, "
          "Tensor lora_t, Tensor lora_u) -> Tensor");
    m.def("quantize_prepack_e5m2(Tensor w, Tensor? ckpt_scale, bool native) -> (Tensor, Tensor)");
    m.def("quantize_prepack_e5m2_scaled(Tensor w, Tensor scale) -> Tensor");
    m.def("lora_down(Tensor x, Tensor d) -> Tensor");
    m.def("bf16_to_fp16(Tensor x, bool rne) -> Tensor");
}

TORCH_LIBRARY_IMPL(feather_ops, CUDA, m) {
    m.impl("scaled_mm", &scaled_mm);
    m.impl("scaled_mm_any_m", &scaled_mm_any_m);
    m.impl("scaled_mm_any_m_lora", &scaled_mm_any_m_lora);
    m.impl("quantize_prepack_e5m2", &quantize_prepack_e5m2);
    m.impl("quantize_prepack_e5m2_scaled", &quantize_prepack_e5m2_scaled);
    m.impl("lora_down", &lora_down);
    m.impl("bf16_to_fp16", &bf16_to_fp16);
}

TORCH_LIBRARY_IMPL(feather_ops, Meta, m) {
    m.impl("scaled_mm_any_m", &scaled_mm_any_m_meta);
    m.impl("scaled_mm_any_m_lora", &scaled_mm_any_m_lora_meta);
    m.impl("lora_down", &lora_down_meta);
    m.impl("bf16_to_fp16", &bf16_to_fp16_meta);
}

// the reference's Python custom op of this name, as a C++ op (the namespace
// also holds the Python-defined autotuned op, so this is a fragment)
TORCH_LIBRARY_FRAGMENT(feather_ops_internal, m) {
    m.def("scaled_mm_configured(Tensor a, Tensor b_prepacked, Tensor? scale, Tensor? bias, ScalarType out_dtype, "
          "int block_warps_m, int block_warps_n, int unroll_k, int repeat_m, int repeat_n) -> Tensor");
}

TORCH_LIBRARY_IMPL(feather_ops_internal, CUDA, m) { m.impl("scaled_mm_configured", &scaled_mm_configured); }

TORCH_LIBRARY_IMPL(feather_ops_internal, Meta, m) { m.impl("scaled_mm_configured", &scaled_mm_configured_meta); }
