// Large-M fp16 x fp8 GEMM on gfx950: LDS-DMA multi-stage pipeline.
//
// Same contract as scaled_mm_tile.hip (reference kernel/hip/hip_kernel.cu:133-420:
// fp32 accumulation, scale on the accumulator, rounding to the output type,
// bias added in the output type) for K % 64 == 0.
//
// Differences from the register-staged tile kernel:
//   * global -> LDS copies use gfx950's global_load_lds_dwordx4: each wave
//     instruction moves 64 x 16 bytes straight into a contiguous 1 KB of LDS,
//     with no VGPR staging and no ds_write. Addresses are a wave-uniform SGPR
//     base (advanced per stage with scalar adds) plus a fixed 32-bit per-lane
//     offset;
//   * A rows are 128 bytes in LDS; chunk c of row r is stored at c ^ swz(r).
//     The swizzle is applied on the global side: the lane that fills LDS chunk
//     p of row r fetches logical chunk p ^ swz(r);
//   * three LDS stage buffers with two stages of copies in flight behind the
//     one being multiplied (the split-K tiles: five or six buffers, four or
//     five stages in flight); each barrier is preceded by an explicit vmcnt
//     wait that leaves the younger stages' copies in flight;
//   * per stage, the K halves are processed one after the other (all M
//     repeats of K half 0, then of K half 1), so only half of the widened B
//     operands are live at a time;
//   * default schedule: the barrier sits early in each stage's second half,
//     after which the next stage's operands can be read while the current
//     stage's remaining MFMAs run (measured on the M=32768 K=5120 N=13824
//     shape: ~5% faster than barrier-at-the-top, which is kept as
//     FEATHEROPS_LDS_PIPE=0). The source asks for A one K half ahead and the
//     copies spread between MFMA groups; the compiler's scheduler keeps the
//     kernel at 255 VGPRs by reading A about one M repeat ahead instead and
//     issues each stage's copies together before the barrier (pinning the
//     source order with scheduling barriers spills, and the other scheduler
//     strategies measured 0-2.5% slower);
//   * rows past M / columns past N are clamped to the last valid row/column
//     (their results are computed and dropped), so every copy is in bounds;
//   * optional rank-R update in the epilogue (kLora, the unmerged LoRA side
//     path of the reference's comfy_feather/lora.py:4-35): after the weight
//     scale, acc += T(M x R) . U(N x R)^T on the fp16 or bf16 MFMA, before
//     the rounding to the output type; the tile's rows of T and U go through
//     the free stage buffers 64 ranks at a time (LDS-DMA, one round trip per
//     64 ranks). The separate pass that would re-read and re-write C
//     disappears.
#include <stdlib.h>

#include <type_traits>

#include "feather_common.h"
#include "lds_dma.h"
#include "scaled_mm_dispatch.h"

namespace feather {
namespace {

// f(std::integral_constant<int, i>{}) for i = 0 .. N-1, in order
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

constexpr int kBK = 64;


// kLora: 0 = none, 1 = fp16 factors, 2 = bf16 factors (T is M x R, U is N x R,
// both row-major with R % 32 == 0 and 16-byte aligned rows)
template <int BM, int BN, int WAVES_M, int WAVES_N, int kPipe, bool kBf16, bool kE4m3, int kLora, int kStages>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void scaled_mm_lds_kernel(
    const uint16_t* __restrict__ A, const uint8_t* __restrict__ Bp, const float* __restrict__ scale,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ C, int M, int N, int K, int has_scale, int has_bias,
    int tiles_m, int tiles_n, int group_m, int ksplit, float* __restrict__ partials, uint32_t* __restrict__ counters,
    const uint16_t* __restrict__ lora_t, const uint16_t* __restrict__ lora_u, int lora_rank, int c_nontemporal) {
    constexpr int kWaves = WAVES_M * WAVES_N;
    constexpr int WTM = BM / WAVES_M;
    constexpr int WTN = BN / WAVES_N;
    constexpr int RM = WTM / 16;
    constexpr int RN = WTN / 16;
    static_assert(WTM % 16 == 0 && WTN % 16 == 0, "wave tile must be a multiple of 16");
    constexpr int kAStage = BM * kBK * 2;
    constexpr int kBStage = BN * kBK;
    constexpr int kStage = kAStage + kBStage;
    constexpr int kAInst = kAStage / 1024;  // 1 KB wave copies per stage
    constexpr int kBInst = kBStage / 1024;
    static_assert(kAInst % kWaves == 0, "A copies must split evenly over waves");
    constexpr int kAPerWave = kAInst / kWaves;
    // B copies are rounded up to a whole number per wave; the surplus slots
    // repeat the last copy (same bytes to the same LDS address), so every
    // wave issues, and waits for, the same number of copies per stage.
    constexpr int kBPerWave = (kBInst + kWaves - 1) / kWaves;
    constexpr int kLoadsPerStage = kAPerWave + kBPerWave;
    static_assert(BN % 64 == 0, "a B copy must stay inside one K group");
    // One LDS object per stage buffer for the first three (the main loop is
    // unrolled by the stage count); deeper rings add buffers behind them.
    static_assert(kStages == 3 || (kPipe == 1 && kStages >= 4 && kStages <= 8), "stage ring depth");
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf0[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf1[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf2[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t sbufx[kStages > 3 ? (kStages - 3) * kStage : 1024];

    // ---- tile index: XCD-contiguous grouped raster; the K splits of a tile
    // are consecutive in that order (so mostly on one XCD) ----
    const int total = tiles_m * tiles_n * ksplit;
    const int pid = blockIdx.x;
    const int xcd = pid % kNumXcd;
    const int per = total / kNumXcd;
    const int rem = total % kNumXcd;
    const int vlin = xcd * per + (xcd < rem ? xcd : rem) + pid / kNumXcd;
    const int lin = vlin / ksplit;
    const int q = vlin - lin * ksplit;
    const int group_size = group_m * tiles_n;
    const int gid = lin / group_size;
    const int first_m = gid * group_m;
    const int gm = (tiles_m - first_m) < group_m ? (tiles_m - first_m) : group_m;
    const int in_group = lin - gid * group_size;
    const int tm = first_m + in_group % gm;
    const int tn = in_group / gm;
    const int m0 = tm * BM;
    const int n0 = tn * BN;

    // The scale, loaded before anything else by a vector load with no branch
    // around it (an absent scale reads A's first bytes and is not used) and
    // selected in the epilogue: it is in long before the epilogue needs it
    // (read there, the scalar load's round trip came before the staging), and
    // as the oldest load it never holds up the stage waits below, which leave
    // only younger copies in flight.
    const uint32_t scale_raw = __builtin_amdgcn_raw_buffer_load_b32(
        __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void*>(has_scale ? static_cast<const void*>(scale) : static_cast<const void*>(A)), 0, 4,
            0x00020000),
        0, 0, 0);
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wave_m = wave % WAVES_M;
    const int wave_n = wave / WAVES_M;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    // K split q covers stages [kt0, kt0 + nk); the host picks ksplit so none is empty
    const int nk_all = K / kBK;
    const int per_split = (nk_all + ksplit - 1) / ksplit;
    const int kt0 = q * per_split;
    const int nk = (nk_all - kt0) < per_split ? (nk_all - kt0) : per_split;

    // ---- per-lane copy offsets (fixed), per-stage SGPR bases ----
    // A copy j of this wave fills rows r0..r0+7 of the tile, r0 = (j * kWaves + wave) * 8.
    uint32_t a_off[kAPerWave];
#pragma unroll
    for (int j = 0; j < kAPerWave; ++j) {
        const int row = (j * kWaves + wave) * 8 + (lane >> 3);
        const int c = (lane & 7) ^ swz(row);
        const int lrow = (m0 + row < M ? m0 + row : M - 1) - m0;
        a_off[j] = static_cast<uint32_t>(lrow * K * 2 + c * 16);
    }
    // B copy j covers chunks [base, base+64) of the (4 x BN) stage, base = b_copy(j) * 64.
    auto b_copy = [&](int j) { return (j * kWaves + wave) < kBInst ? (j * kWaves + wave) : kBInst - 1; };
    uint32_t b_off[kBPerWave];
#pragma unroll
    for (int j = 0; j < kBPerWave; ++j) {
        const int chunk = b_copy(j) * 64 + lane;
        const int kb = chunk / BN;
        const int lcol = (n0 + chunk % BN < N ? n0 + chunk % BN : N - 1) - n0;
        b_off[j] = static_cast<uint32_t>((kb * N + lcol) * 16);
    }
    const int64_t b_stage_bytes = static_cast<int64_t>(N) * 64;  // 4 K groups of N x 16 bytes
    const uint8_t* a_base = reinterpret_cast<const uint8_t*>(A) + static_cast<int64_t>(m0) * K * 2 + kt0 * (kBK * 2);
    const uint8_t* b_base = Bp + static_cast<int64_t>(n0) * 16 + kt0 * b_stage_bytes;

    auto stage_buf = [&](auto tag) -> uint8_t* {
        constexpr int b = decltype(tag)::value;
        if constexpr (b == 0) return sbuf0;
        else if constexpr (b == 1) return sbuf1;
        else if constexpr (b == 2) return sbuf2;
        else return sbufx + (b - 3) * kStage;
    };
    // LDS byte address of stage buffer `tag` (a constant)
    auto stage_lds = [&](auto tag) -> uint32_t { return lds_addr_of(stage_buf(tag)); };
    // copy i (A copies first, then B copies) of stage kt into buffer `tag`
    auto issue_one = [&](auto tag, int kt, int i) {
        const uint32_t la = stage_lds(tag);
        if (i < kAPerWave) {
            dma16_lds(a_base + kt * (kBK * 2), a_off[i], la + ((i * kWaves + wave) * 8) * 128);
        } else {
            const int j = i - kAPerWave;
            dma16_lds(b_base + kt * b_stage_bytes, b_off[j], la + kAStage + (b_copy(j) * 64) * 16);
        }
    };
    auto issue_stage = [&](auto tag, int kt) {
#pragma unroll
        for (int i = 0; i < kLoadsPerStage; ++i) issue_one(tag, kt, i);
    };
    // LDS byte offset of this lane's A operand for M repeat rm, K half kh
    auto a_lds = [&](int rm, int kh) -> int {
        const int row = wave_m * WTM + rm * 16 + lr;
        return row * 128 + (((2 * lg + kh) ^ swz(row)) << 4);
    };
    // operand reads as LDS byte addresses: a constant per buffer (and M / N
    // repeat) plus one per-lane offset, so the constants can sit in the
    // ds_read offset field instead of in extra address registers
    auto lds_ld16 = [](uint32_t addr) -> uint4 {
        using v4 = uint32_t __attribute__((ext_vector_type(4)));
        const v4 v = *reinterpret_cast<const __attribute__((address_space(3))) v4*>(static_cast<uintptr_t>(addr));
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    const uint32_t b_lane = static_cast<uint32_t>((lg * BN + wave_n * WTN + lr) * 16);
    const uint32_t a_lane0 = static_cast<uint32_t>(a_lds(0, 0));
    const uint32_t a_lane1 = static_cast<uint32_t>(a_lds(0, 1));
    auto read_b = [&](auto cur, uint4 (&braw)[RN]) {
        const uint32_t sb = stage_lds(cur) + kAStage + b_lane;
#pragma unroll
        for (int rn = 0; rn < RN; ++rn) braw[rn] = lds_ld16(sb + rn * 256);
    };

    f32x4 acc[RM][RN];
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
        for (int j = 0; j < RN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;

    // A fragments of one K half of a stage, for every M repeat
    // (the A swizzle depends on row & 15 only, so M repeat rm adds rm * 16 rows)
    auto read_a = [&](auto tag, int kh, uint4 (&dst)[RM]) {
        const uint32_t sa = stage_lds(tag) + (kh ? a_lane1 : a_lane0);
#pragma unroll
        for (int rm = 0; rm < RM; ++rm) dst[rm] = lds_ld16(sa + rm * 16 * 128);
    };
    // MFMAs of one K half: widen this half of the B operands, then run every
    // M repeat; `hook(rm)` runs before the MFMAs of repeat rm. The widened
    // weights are the MFMA's first operand and the activations its second, so
    // each 16x16 result is C^T: lane (lr, lg) element i is C[row lr][col
    // 4*lg + i] of the tile. Measured 1.8% faster than the other operand order
    // on M=32768 N=13824 K=5120 (the kernel is power-bound with random data).
    // Changing the activation operand costs more than changing the weight
    // operand (an e5m2 byte widens to an fp16 with a zero low byte): running the M
    // repeats innermost measured 4% slower.
    // Pinned schedule (default schedule, wave tiles of at least 64 x 64):
    // each weight column is widened just before it is first needed, in
    // program order with the MFMAs (both inline asm, so neither moves), instead
    // of a whole K half's columns in one burst ahead of its first MFMA; the
    // MFMAs run in a serpentine over the columns, and the next K half's first
    // two columns are widened during this half's last repeat once they are
    // free. Medians of alternating runs on MI355X, the same bits: M=32768
    // N=13824 K=5120 (256 x 256, 4 x 2 waves) 3.268 vs 3.315 ms, 8192^3 0.765
    // vs 0.774 ms; M=4096 N=3072 K=3072 (128 x 384) 56.2 vs 57.8 us, K=12288
    // 209.8 vs 213.7 us (256 x 192 on 4 x 2 waves: 210.3 vs 217.1 us on 2 x 4);
    // M=2048 N=K=4096: 128 x 256 52.0 vs 52.8 us, 256 x 128 53.3 vs 54.9 us,
    // 128 x 128 62.9 vs 63.6 us; e4m3fn weights at M=32768 N=13824 K=5120
    // 3.225 vs 3.251 ms (4 x 2 pinned vs 2 x 4 compiler-scheduled). Ordering
    // rules the asm keeps by construction (the compiler's hazard tracking does
    // not see inside asm): a widened column is written at least two MFMAs
    // before an MFMA reads it (the register of one an MFMA has read may be
    // rewritten right after it, as the compiler's own code for builtin MFMAs
    // does), the MFMAs accumulate in place with nothing else touching the
    // accumulators in the loop, and other instructions read the accumulators
    // only after the wait states that follow the main loop (all checked on the
    // compiled code by tests/test_pinned_codegen.py).
    constexpr bool kPinned = kPipe == 1 && RM % 2 == 0 && RM >= 4 && RN >= 4;
    // widen_fp8x8's instructions as asm (e5m2: byte shuffles; e4m3fn: the
    // hardware fp8 -> fp16 conversion with scale 1, low then high word)
    auto widen_pinned = [](uint32_t lo, uint32_t hi) -> half8_t {
        uint32_t w0, w1, w2, w3;
        if constexpr (!kE4m3) {
            asm volatile(
                "v_perm_b32 %0, 0, %4, %6\n\t"
                "v_perm_b32 %1, 0, %4, %7\n\t"
                "v_perm_b32 %2, 0, %5, %6\n\t"
                "v_perm_b32 %3, 0, %5, %7"
                : "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3)
                : "v"(lo), "v"(hi), "s"(0x010c000cu), "s"(0x030c020cu));
        } else {
            asm volatile(
                "v_cvt_scalef32_pk_f16_fp8 %0, %4, 1.0\n\t"
                "v_cvt_scalef32_pk_f16_fp8 %1, %4, 1.0 op_sel:[1,0,0]\n\t"
                "v_cvt_scalef32_pk_f16_fp8 %2, %5, 1.0\n\t"
                "v_cvt_scalef32_pk_f16_fp8 %3, %5, 1.0 op_sel:[1,0,0]"
                : "=&v"(w0), "=&v"(w1), "=&v"(w2), "=&v"(w3)
                : "v"(lo), "v"(hi));
        }
        return __builtin_bit_cast(half8_t, make_uint4(w0, w1, w2, w3));
    };
    half8_t bqp[RN];  // pinned schedule: the current K half's widened columns
    auto mm_half = [&](int kh, const uint4 (&araw)[RM], const uint4 (&braw)[RN], auto hook, bool pre = false) {
        if constexpr (kPinned) {
            // MFMA j of repeat rm uses column col(kh, rm, j): forward or
            // reversed by repeat, K half 1 starting reversed, so the columns the
            // next half needs first are the ones this half's last repeat uses
            // first. pre: widen the next half's first two columns here (braw
            // holds the next stage's weights by then when kh == 1).
            auto col = [](int h, int rm, int j) { return (((rm & 1) ^ h) != 0) ? RN - 1 - j : j; };
            auto wd = [&](int rn, int h) {
                bqp[rn] = h == 0 ? widen_pinned(braw[rn].x, braw[rn].y) : widen_pinned(braw[rn].z, braw[rn].w);
            };
            constexpr int kPre = RN >= 6 ? RN / 2 : 2;
#pragma unroll
            for (int rm = 0; rm < RM; ++rm) {
                hook(rm);
                const half8_t a = a_frag<false>(araw[rm]);
#pragma unroll
                for (int j = 0; j < RN; ++j) {
                    if (rm == 0 && j + 2 < RN) wd(col(kh, 0, j + 2), kh);
                    if (rm == RM - 1 && pre && (j == kPre || j == kPre + 1)) wd(col(kh ^ 1, 0, j - kPre), kh ^ 1);
                    const int rn = col(kh, rm, j);
                    f32x4 t = acc[rm][rn];
                    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(t) : "v"(bqp[rn]), "v"(a));
                    acc[rm][rn] = t;
                }
            }
            return;
        }
        half8_t bq[RN];
#pragma unroll
        for (int rn = 0; rn < RN; ++rn)
            bq[rn] = kh == 0 ? widen_fp8x8<kE4m3>(braw[rn].x, braw[rn].y) : widen_fp8x8<kE4m3>(braw[rn].z, braw[rn].w);
#pragma unroll
        for (int rm = 0; rm < RM; ++rm) {
            hook(rm);
            const half8_t a = a_frag<false>(araw[rm]);
#pragma unroll
            for (int j = 0; j < RN; ++j) {
                // serpentine over the N repeats: consecutive MFMAs change only
                // one operand (0.6-1.5% faster on M=32768 N=13824 K=5120 than
                // restarting at rn = 0; again a power effect)
                const int rn = (rm & 1) ? RN - 1 - j : j;
                acc[rm][rn] = mfma16x16x32(bq[rn], a, acc[rm][rn]);
            }
        }
    };

    if constexpr (kPipe == 1) {
        // Operands one K half ahead (as written; see the file header for what
        // the scheduler makes of it). Register set araw[kh] holds the A
        // fragments of K half kh of the current stage: the second half's are
        // requested at the start of the first half's MFMAs. Stage kt + 2's
        // copies are placed between the first half's M repeats. Early in the
        // second half -- once every wave has all of stage kt in registers --
        // a barrier publishes stage kt + 1 (its copies were waited for just
        // before) and frees stage kt's buffer, and stage kt + 1's first-half
        // operands are requested while the remaining repeats run.
        constexpr int kBarrierRm = RM / 4;
        uint4 araw[2][RM];
        uint4 braw[RN];
        // Deeper rings (kStages > 3) always keep kStages - 1 stages of copies
        // issued: a stage past the end copies stage nk - 1 again into its
        // (never read) buffer, so every wait count is a constant and no
        // branch surrounds a copy; the main loop waits for those copies
        // before the epilogue reuses the buffers.
        issue_stage(S0{}, 0);
        if constexpr (kStages == 3) {
            if (nk > 1) {
                issue_stage(S1{}, 1);
                wait_vmcnt<kLoadsPerStage>();
            } else {
                wait_vmcnt<0>();
            }
        } else {
            static_for<kStages - 2>([&](auto i) {
                constexpr int st = decltype(i)::value + 1;
                issue_stage(std::integral_constant<int, st>{}, st < nk ? st : nk - 1);
            });
            wait_vmcnt<(kStages - 2) * kLoadsPerStage>();
        }
        stage_barrier();
        read_b(S0{}, braw);
        read_a(S0{}, 0, araw[0]);
        if constexpr (kPinned) {
            // K half 0 of stage 0 starts forward: columns 0 and 1
            static_assert(RM / 4 >= 1, "the next stage's weights arrive after repeat 0");
            bqp[0] = widen_pinned(braw[0].x, braw[0].y);
            bqp[1] = widen_pinned(braw[1].x, braw[1].y);
        }
        // kFull (three-stage ring): stages kt + 1 and kt + 2 exist (no bounds
        // checks, so the steady-state loop body has no branches around the
        // copies; a checked copy of the loop runs the last three to five
        // stages). Deeper rings run every stage unchecked, the copies of
        // stages past the end clamped to the last one.
        auto run_stage = [&](auto cur, auto full, int kt) {
            constexpr int c = decltype(cur)::value;
            constexpr bool kFull = decltype(full)::value;
            using Next = std::integral_constant<int, (c + 1) % kStages>;
            // stage kt + kStages - 1's buffer (stage kt - 1's, freed by its barrier)
            using Free = std::integral_constant<int, (c + kStages - 1) % kStages>;
            const bool has2 = kStages > 3 || kFull || kt + 2 < nk;
            const bool has1 = kStages > 3 || kFull || kt + 1 < nk;
            const int kt_free = kStages > 3 && kt + kStages - 1 >= nk ? nk - 1 : kt + kStages - 1;
            mm_half(0, araw[0], braw, [&](int rm) {
                if (rm == 0) read_a(cur, 1, araw[1]);
#pragma unroll
                for (int i = 0; i < kLoadsPerStage; ++i)
                    if (rm == (i * RM) / kLoadsPerStage && has2) issue_one(Free{}, kt_free, i);
            }, true);
            // mm_half widens braw before the first hook, so the hook may
            // overwrite braw with the next stage's operands
            mm_half(1, araw[1], braw, [&](int rm) {
                if (rm == kBarrierRm && has1) {
                    // this wave's reads of stage kt have returned, stage kt + 1 has landed
                    if (has2) wait_vmcnt_lgkm0<(kStages - 2) * kLoadsPerStage>();
                    else wait_vmcnt_lgkm0<0>();
                    stage_barrier();
                    read_b(Next{}, braw);
                    read_a(Next{}, 0, araw[0]);
                }
            }, has1);
        };
        using Full = std::true_type;
        using Tail = std::false_type;
        int kt = 0;
        if constexpr (kStages == 3) {
            for (; kt + 5 <= nk; kt += 3) {
                run_stage(S0{}, Full{}, kt);
                run_stage(S1{}, Full{}, kt + 1);
                run_stage(S2{}, Full{}, kt + 2);
            }
            for (; kt < nk; kt += 3) {
                run_stage(S0{}, Tail{}, kt);
                if (kt + 1 < nk) run_stage(S1{}, Tail{}, kt + 1);
                if (kt + 2 < nk) run_stage(S2{}, Tail{}, kt + 2);
            }
        } else {
            for (; kt + kStages <= nk; kt += kStages)
                static_for<kStages>([&](auto c) { run_stage(c, Full{}, kt + decltype(c)::value); });
            static_for<kStages>([&](auto c) {
                if (kt + decltype(c)::value < nk) run_stage(c, Full{}, kt + decltype(c)::value);
            });
            wait_vmcnt<0>();  // the repeated copies past the end
        }
    } else {
        // Plain schedule: at the top of stage kt wait for its copies (issued
        // two stages earlier), barrier, issue stage kt + 2's copies into the
        // buffer stage kt - 1 used, then read and multiply both K halves.
        auto no_hook = [](int) {};
        auto run_stage = [&](auto cur, int kt) {
            constexpr int c = decltype(cur)::value;
            using Free = std::integral_constant<int, (c + 2) % 3>;
            if (kt + 1 < nk) wait_vmcnt<kLoadsPerStage>();
            else wait_vmcnt<0>();
            stage_barrier();
            if (kt + 2 < nk) issue_stage(Free{}, kt + 2);
            uint4 braw[RN];
            read_b(cur, braw);
            uint4 araw[RM];
            read_a(cur, 0, araw);
            mm_half(0, araw, braw, no_hook);
            read_a(cur, 1, araw);
            mm_half(1, araw, braw, no_hook);
        };
        issue_stage(S0{}, 0);
        if (nk > 1) issue_stage(S1{}, 1);
        for (int kt = 0; kt < nk; kt += 3) {
            run_stage(S0{}, kt);
            if (kt + 1 < nk) run_stage(S1{}, kt + 1);
            if (kt + 2 < nk) run_stage(S2{}, kt + 2);
        }
    }

    // pinned schedule: wait states between the last asm MFMA and any other
    // instruction that reads its accumulator
    if constexpr (kPinned) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    // the scale into a scalar register here, where the main loop has already
    // waited for every load (the memory clobber keeps the epilogue's bias load
    // from being issued before this wait, so the bias still lands behind the
    // staging writes)
    uint32_t scale_s;
    asm volatile("v_readfirstlane_b32 %0, %1" : "=s"(scale_s) : "v"(scale_raw) : "memory");
    const float s = has_scale ? __uint_as_float(scale_s) : 1.0f;
    // (K split: only the 32- and 64-row tiles are ever launched with ksplit > 1)
    if constexpr (BM <= 64) if (ksplit > 1) {
        // ---- K split: each workgroup writes its fp32 accumulators to the
        // workspace in fragment order (lane-contiguous 16-byte pieces) and
        // bumps the tile's arrival counter; the workgroup that arrives last
        // adds the ksplit partials in split order (deterministic), then runs
        // the normal epilogue and re-zeroes the counter.
        // Ordering: the partials are only ever written and read with agent-scope
        // (sc1) accesses -- the instructions the AMDGPU memory model uses for
        // relaxed agent-scope atomic stores and loads on gfx942/gfx950 -- so
        // they are coherent across XCDs without any L2 write-back or
        // invalidate. A store is acknowledged (vmcnt) only once it is visible
        // at agent scope; every wave waits for that before the barrier, and
        // the arrival RMW is issued after the barrier, so it follows every
        // partial of this workgroup. The last arrival's loads are issued after
        // the RMW has returned (they depend on last_flag through LDS and a
        // barrier) and read the coherence point directly. An agent-scope
        // release/acquire pair instead costs an L2 write-back and invalidate
        // per workgroup (measured: M=64 N=13824 K=5120 25 -> 38 us).
        constexpr int kTileBytes = BM * BN * 4;
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            partials + static_cast<int64_t>(lin) * ksplit * (kTileBytes / 4), 0, ksplit * kTileBytes, 0x00020000);
        auto frag_off = [&](int rm, int rn) { return (((wave * RM + rm) * RN + rn) * 64 + lane) * 16; };
        constexpr int kCoherent = 16;  // sc1
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int rm = 0; rm < RM; ++rm)
#pragma unroll
            for (int rn = 0; rn < RN; ++rn)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[rm][rn]), prs,
                                                       q * kTileBytes + frag_off(rm, rn), 0, kCoherent);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partial stores are acknowledged
        __shared__ int last_flag;
        __syncthreads();
        if (tid == 0)
            last_flag = __hip_atomic_fetch_add(&counters[lin], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        static_cast<uint32_t>(ksplit - 1);
        __syncthreads();
        if (!last_flag) return;
        // the partials are re-read in split order, kQ splits' loads in flight at a time
        constexpr int kQ = RM * RN <= 4 ? 4 : RM * RN <= 8 ? 2 : 1;
#pragma unroll
        for (int rm = 0; rm < RM; ++rm)
#pragma unroll
            for (int rn = 0; rn < RN; ++rn) acc[rm][rn] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int q0 = 0; q0 < ksplit; q0 += kQ) {
            f32x4 t[kQ][RM][RN];
#pragma unroll
            for (int j = 0; j < kQ; ++j)
#pragma unroll
                for (int rm = 0; rm < RM; ++rm)
#pragma unroll
                    for (int rn = 0; rn < RN; ++rn)
                        t[j][rm][rn] = q0 + j < ksplit
                                           ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                           prs, (q0 + j) * kTileBytes + frag_off(rm, rn),
                                                                           0, kCoherent))
                                           : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kQ; ++j)
#pragma unroll
                for (int rm = 0; rm < RM; ++rm)
#pragma unroll
                    for (int rn = 0; rn < RN; ++rn) acc[rm][rn] += t[j][rm][rn];
        }
        if (tid == 0)  // ready for the next call on this stream
            __hip_atomic_store(&counters[lin], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    if constexpr (kLora != 0) {
        // the weight scale applies to the fp8 product only: scale first, then
        // add the rank-R term in fp32 (one MFMA K step per 32 ranks; weights'
        // role for U, activations' role for T, so the accumulator layout is
        // the main loop's)
        static_assert(kStage >= BM * 128 && kStage >= BN * 128, "a 64-rank chunk of T or U must fit a stage buffer");
#pragma unroll
        for (int rm = 0; rm < RM; ++rm)
#pragma unroll
            for (int rn = 0; rn < RN; ++rn)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[rm][rn][i] = opaque_f32(acc[rm][rn][i] * s);
        // 64 ranks at a time, the tile's T rows and U rows are copied into the
        // (now free) stage buffers with the A operand's layout (128-byte rows,
        // chunk c at c ^ swz(row)), one round trip for the whole tile, and the
        // MFMA steps read their fragments from LDS. Step kh covers ranks
        // [32 kh, 32 kh + 32): lane group lg reads chunk lg + 4 kh of T and U.
        // A 32-rank tail copies ranks [0, 32) only and runs step 0.
        const uint32_t lt = lds_addr_of(sbuf0);
        const uint32_t lu = lds_addr_of(sbuf1);
        constexpr int kTInst = BM / 8;  // 1 KB copies: 8 rows of 64 ranks
        constexpr int kUInst = BN / 8;
        for (int r0 = 0; r0 < lora_rank; r0 += 64) {
            const bool tail = lora_rank - r0 < 64;
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the buffers are done
            stage_barrier();                      // and every other wave's
            for (int j = wave; j < kTInst + kUInst; j += kWaves) {
                const bool is_t = j < kTInst;
                const int jj = is_t ? j : j - kTInst;
                const int row = jj * 8 + (lane >> 3);
                int c = (lane & 7) ^ swz(row);
                if (tail && c >= 4) c -= 4;  // past the rank: a valid chunk, never read
                const int grow = is_t ? (m0 + row < M ? m0 + row : M - 1) : (n0 + row < N ? n0 + row : N - 1);
                dma16_lds(is_t ? lora_t : lora_u, static_cast<uint32_t>((grow * lora_rank + r0 + 8 * c) * 2),
                          (is_t ? lt : lu) + jj * 1024);
            }
            wait_vmcnt<0>();
            stage_barrier();
            for (int kh = 0; kh < (tail ? 1 : 2); ++kh) {
                uint4 tf[RM], uf[RN];
#pragma unroll
                for (int rm = 0; rm < RM; ++rm) {
                    const int row = wave_m * WTM + rm * 16 + lr;
                    tf[rm] = lds_ld16(lt + row * 128 + (((lg + 4 * kh) ^ swz(row)) << 4));
                }
#pragma unroll
                for (int rn = 0; rn < RN; ++rn) {
                    const int row = wave_n * WTN + rn * 16 + lr;
                    uf[rn] = lds_ld16(lu + row * 128 + (((lg + 4 * kh) ^ swz(row)) << 4));
                }
#pragma unroll
                for (int rm = 0; rm < RM; ++rm)
#pragma unroll
                    for (int rn = 0; rn < RN; ++rn) {
                        if constexpr (kLora == 1)
                            acc[rm][rn] = mfma16x16x32(as_half8(uf[rn]), as_half8(tf[rm]), acc[rm][rn]);
                        else
                            acc[rm][rn] = mfma16x16x32_bf16(uf[rn], tf[rm], acc[rm][rn]);
                    }
            }
        }
    }

    // ---- epilogue: each wave stages its whole WTM x WTN output tile in LDS
    // (the stage buffers, free once every wave is past its last stage) with
    // one wait, then stores rows of WTN * 2 contiguous bytes ----
    const int out_col0 = n0 + wave_n * WTN;
    constexpr int kCPR = WTN / 8;                // 16-byte chunks per staged row
    constexpr int kRowBytes = WTN * 2;
    constexpr int kRowsPerStore = 64 / kCPR;     // rows one store instruction covers
    constexpr int kLanesUsed = kRowsPerStore * kCPR;
    constexpr int kWaveBytes = WTM * kRowBytes;
    constexpr int kWavesPerBuf = kStage / kWaveBytes;
    static_assert(3 * kWavesPerBuf >= kWaves, "epilogue staging must fit the stage buffers");
    const int cc = lane % kCPR;  // this lane's chunk of every row it stores
    const int rsub = lane / kCPR;
    const int gcol = out_col0 + cc * 8;
    // the bias chunk is issued before the barrier and waited for after the
    // staging writes, so its latency overlaps them
    const uint4 b8 = has_bias && lane < kLanesUsed && gcol < N ? load_bias8(bias + gcol) : make_uint4(0u, 0u, 0u, 0u);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's last operand reads are done
    stage_barrier();
    uint8_t* sc = (wave / kWavesPerBuf == 0 ? sbuf0 : wave / kWavesPerBuf == 1 ? sbuf1 : sbuf2) +
                  (wave % kWavesPerBuf) * kWaveBytes;
    // chunk c of staged row r sits at (c + r) % kCPR (spreads the rows of one
    // write over the LDS banks). bf16 outputs are converted without NaN
    // canonicalisation first; a wave that produced a NaN stages again with
    // torch's canonical NaN (the per-pair canonicalisation in staging and in
    // the bias add cost ~0.7 us per tile: M=4096 N=3072 K=3072 57.9 -> 56.5 us).
    uint32_t nan_track = 0u;
    auto stage = [&](auto canonical) {
        constexpr bool kCanon = decltype(canonical)::value;
#pragma unroll
        for (int rm = 0; rm < RM; ++rm) {
            const int row = rm * 16 + lr;
#pragma unroll
            for (int rn = 0; rn < RN; ++rn) {
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[i] = kLora != 0 ? acc[rm][rn][i]
                                      : opaque_f32(acc[rm][rn][i] * s);
                // row lr, columns 4*lg .. 4*lg+3 of this 16x16 tile: one 8-byte write
                const int chunk = (2 * rn + (lg >> 1) + row) % kCPR;
                uint32_t w0, w1;
                if constexpr (kBf16 && !kCanon) {
                    w0 = f32x2_to_bf16x2_raw(v[0], v[1]);
                    w1 = f32x2_to_bf16x2_raw(v[2], v[3]);
                    nan_track = bf16x2_nan_track(bf16x2_nan_track(nan_track, w0), w1);
                } else {
                    w0 = f32x2_to_out_bits<kBf16>(v[0], v[1]);
                    w1 = f32x2_to_out_bits<kBf16>(v[2], v[3]);
                }
                *reinterpret_cast<uint2*>(sc + row * kRowBytes + chunk * 16 + (lg & 1) * 8) = make_uint2(w0, w1);
            }
        }
    };
    stage(std::false_type{});
    if constexpr (kBf16)
        if (__builtin_amdgcn_ballot_w64(bf16x2_nan_seen(nan_track))) stage(std::true_type{});
    // staging writes and the bias load complete: one wait, then no vmcnt wait
    // between the stores (vmcnt counts stores too)
    __builtin_amdgcn_s_waitcnt(0x0070);  // vmcnt(0) lgkmcnt(0)
    wave_lds_sync();                     // each wave reads only its own region
    const int out_row0 = m0 + wave_m * WTM;
#pragma unroll
    for (int p = 0; p < (WTM + kRowsPerStore - 1) / kRowsPerStore; ++p) {
        const int r = p * kRowsPerStore + rsub;
        const int grow = out_row0 + r;
        if (lane < kLanesUsed && r < WTM && grow < M && gcol < N) {
            uint4 v = *reinterpret_cast<const uint4*>(sc + r * kRowBytes + ((cc + r) % kCPR) * 16);
            if (has_bias) {
                if constexpr (kBf16) {
                    uint4 vb = v;
                    uint32_t nt = 0u;
                    add_bias8<true, false>(vb, b8, &nt);
                    if (__builtin_amdgcn_ballot_w64(bf16x2_nan_seen(nt))) add_bias8<true>(v, b8);
                    else v = vb;
                } else {
                    add_bias8<false>(v, b8);
                }
            }
            uint4* dst = reinterpret_cast<uint4*>(C + static_cast<int64_t>(grow) * N + gcol);
            if (c_nontemporal) {
                typedef uint32_t u32x4_nt __attribute__((ext_vector_type(4)));
                __builtin_nontemporal_store(u32x4_nt{v.x, v.y, v.z, v.w}, reinterpret_cast<u32x4_nt*>(dst));
            } else {
                *dst = v;
            }
        }
    }
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int PIPE, int STAGES = 3>
bool launch_lds(const MmArgs& p, hipStream_t stream, int ksplit = 1, float* partials = nullptr,
                uint32_t* counters = nullptr) {
    const int tiles_m = (p.M + BM - 1) / BM;
    const int tiles_n = (p.N + BN - 1) / BN;
    const int group_m = p.group_m > 0 ? p.group_m : 4;
    // Outputs larger than the 256 MB MALL are written with nontemporal stores:
    // they are never re-read here and cannot stay cached for the next layer
    // anyway (M=32768 N=13824 K=5120 3.096 -> 3.081 ms on MI355X). Smaller
    // outputs keep ordinary stores: nontemporal ones measured ~2% faster for an
    // isolated one-wave M=4096 N=3072 GEMM, but a chained FFN (M=4096,
    // 3072 -> 12288 -> 3072) took 414 us with ordinary stores and 419 us with
    // the 100 MB intermediate written nontemporally.
    const int c_nt = p.M * p.N * 2 > (int64_t(256) << 20) ? 1 : 0;
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n * ksplit));
    const dim3 block(64 * WAVES_M * WAVES_N);
#define FEATHER_LDS_LAUNCH_L(BF, E4, LORA)                                                                            \
    hipLaunchKernelGGL((scaled_mm_lds_kernel<BM, BN, WAVES_M, WAVES_N, PIPE, BF, E4, LORA, STAGES>), grid, block, 0,          \
                       stream, p.a, p.b, p.scale, p.bias, p.c, static_cast<int>(p.M), static_cast<int>(p.N),          \
                       static_cast<int>(p.K), p.has_scale, p.has_bias, tiles_m, tiles_n, group_m, ksplit, partials,   \
                       counters, p.lora_t, p.lora_u, static_cast<int>(p.lora_rank), c_nt)
#define FEATHER_LDS_LAUNCH(BF, E4) FEATHER_LDS_LAUNCH_L(BF, E4, 0)
    if (p.lora_dtype != 0) {
        // rank-R epilogue: the default schedule's large tiles, fp16 activations,
        // e5m2 weights, no K split
        // (the T and U chunks must fit a stage buffer: not the 128 x 384 tile)
        if constexpr (PIPE == 1 && BM >= 128 && BM * 128 + BN * 64 >= (BM > BN ? BM : BN) * 128) {
            if (p.a_bf16 || p.b_e4m3 || ksplit != 1) return false;
            if (p.lora_dtype == 1) {
                if (p.out_bf16) FEATHER_LDS_LAUNCH_L(true, false, 1);
                else FEATHER_LDS_LAUNCH_L(false, false, 1);
            } else {
                if (p.out_bf16) FEATHER_LDS_LAUNCH_L(true, false, 2);
                else FEATHER_LDS_LAUNCH_L(false, false, 2);
            }
            return true;
        }
        return false;
    }
    // bf16 activations: none of these tiles; the caller rounds A to fp16 first.
    // Converting each A fragment as it is read costs more than a separate cast
    // pass on every tile here, because each fragment is read by 2-4 waves and
    // feeds only 1-6 MFMAs (graph-replayed, bf16 out, M=512 N=3072 K=12288 on
    // the 64 x 64 split-K tiles: 102 us converted in the kernel vs 60 us cast
    // first, fp16 A 54 us; M=4096 N=3072 K=3072 on the 128 x 384 tile: 68 vs
    // 66 us; M=32768 N=13824 K=5120 on the 256 x 256 tile: 4.44 vs 3.68 ms).
    if (p.a_bf16) return false;
    if (p.out_bf16) {
        if (p.b_e4m3) FEATHER_LDS_LAUNCH(true, true);
        else FEATHER_LDS_LAUNCH(true, false);
    } else {
        if (p.b_e4m3) FEATHER_LDS_LAUNCH(false, true);
        else FEATHER_LDS_LAUNCH(false, false);
    }
#undef FEATHER_LDS_LAUNCH
#undef FEATHER_LDS_LAUNCH_L
    return true;
}

template <int PIPE>
bool launch_lds_pipe(int kernel_id, const MmArgs& p, hipStream_t stream, int ks = 1, float* partials = nullptr,
                     uint32_t* counters = nullptr, int stages = 3) {
    switch (kernel_id) {
        // 256 x 256 and 256 x 192 on 4 x 2 waves (64 x 128 / 64 x 96 wave tiles:
        // 20% fewer LDS operand bytes per stage than 2 x 4, and wide enough
        // for the pinned schedule)
        case kLds256x256: return launch_lds<256, 256, 4, 2, PIPE>(p, stream);
        case kLds256x128: return launch_lds<256, 128, 4, 2, PIPE>(p, stream);
        case kLds128x256: return launch_lds<128, 256, 2, 4, PIPE>(p, stream);
        case kLds128x128: return launch_lds<128, 128, 2, 2, PIPE>(p, stream);
        case kLds256x192: return launch_lds<256, 192, 4, 2, PIPE>(p, stream);
        case kLds128x384: return launch_lds<128, 384, 2, 4, PIPE>(p, stream);
        // default schedule: a five- or six-stage ring (see lds_splitk_plan)
#define FEATHER_SK(BM_, BN_)                                                                             \
    if constexpr (PIPE == 1) {                                                                           \
        if (stages == 6) return launch_lds<BM_, BN_, 1, 4, PIPE, 6>(p, stream, ks, partials, counters); \
        return launch_lds<BM_, BN_, 1, 4, PIPE, 5>(p, stream, ks, partials, counters);                  \
    } else {                                                                                             \
        return launch_lds<BM_, BN_, 1, 4, PIPE>(p, stream, ks, partials, counters);                     \
    }
        case kLdsSk64x64: FEATHER_SK(64, 64);
        case kLdsSk64x128: FEATHER_SK(64, 128);
        case kLdsSk32x128: FEATHER_SK(32, 128);
#undef FEATHER_SK
        default: return false;
    }
}

}  // namespace

int lds_pipe_env() {
    // FEATHEROPS_LDS_PIPE: 1 (default) = operand-prefetch schedule, 0 = plain schedule
    static const int pipe_env = [] {
        const char* e = getenv("FEATHEROPS_LDS_PIPE");
        return e ? atoi(e) : 1;
    }();
    return pipe_env;
}

bool launch_lds_kernel(int kernel_id, const MmArgs& p, hipStream_t stream) {
    if (p.K % kBK != 0) return false;
    return lds_pipe_env() == 0 && !p.a_bf16 && p.lora_dtype == 0 ? launch_lds_pipe<0>(kernel_id, p, stream)
                                                                 : launch_lds_pipe<1>(kernel_id, p, stream);
}

// Split-K plan for the 32- and 64-row tiles: as many K splits as keep the
// grid within `target` workgroups (each split keeps at least one 64-K stage;
// no split below 32 stages), and the stage ring's depth.
// Measured on MI355X (weights rotated past the MALL): 64 x 64 tiles beat
// 64 x 128 / 64 x 256 at M = 64 for N = 3072..13824, and 32 x 128 is the best
// 32-row tile (the small-M kernel still wins at M <= 32).
// Stage ring and grid (back to back, us, 3 / 5 / 6 stages at the grid this
// plan picks): M=64 N=13824 K=5120 (216 tiles, one split) 31.1 / 20.9 / 20.8;
// M=64 N=3072 K=12288 (4 splits) 22.1 / 15.9 / 15.8; M=40 N=13824 K=5120
// 31.0 / 19.4 / 18.6; M=256 N=3072 K=3072 13.4 / 10.2 / 10.4; M=256
// N=K=1024 5.60 / 5.18 / 5.37; M=1024 N=K=1024 6.84 / 5.69 / 5.82. The
// three-stage ring did best with about twice the workgroups (two splits of
// M=64 N=13824 K=5120: 24.9 us), with which the deeper rings lose (25.5):
// one workgroup per CU with five or six stages of copies in flight streams
// better than two sharing a CU with two each, and saves the partial-sum
// round trip.
SplitKPlan lds_splitk_plan(int64_t M, int64_t N, int64_t K, int target) {
    SplitKPlan pl{};
    if (M <= 0 || K % kBK != 0) return pl;
    const int bm = M <= 32 ? 32 : 64;
    const int64_t nk = K / kBK;
    auto splits = [&](int64_t tiles) {
        int64_t ks = target / tiles;
        // below 32 stages (K < 2048) the split's partial round trip costs more than the stages it
        // spreads (measured: M=256 N=K=1024 6.0 us unsplit vs 7.2 us in 4 splits, M=256 N=2048
        // K=512 4.7 vs 6.7 us; from K=2048 on splitting wins or ties)
        if (nk < 32) ks = 1;
        if (ks > nk) ks = nk;
        if (ks > 32) ks = 32;
        if (ks < 1) ks = 1;
        const int64_t per = (nk + ks - 1) / ks;
        ks = (nk + per - 1) / per;  // no empty split
        if (tiles > kWorkspaceCounters) ks = 1;  // more tiles than the counter region holds
        return ks;
    };
    // 64 rows: 64 x 64 tiles, or 64 x 128 where their grid comes closer to
    // `target` without passing it (or, past it, is smaller) in at most four K
    // splits. The last workgroup of a tile re-reads every split's partial
    // tile (32 KB at 64 x 128), so many splits of wide tiles lose: M=64 N=K=4096
    // (256 workgroups either way) 8.9 us on 64 x 64, 12.4 us on 64 x 128;
    // M=64 N=2176 K=8128 (238 workgroups in 7 splits vs 255 in 15) 10.6 vs
    // 17.1 us; M=64 N=6144 K=4096 (192 in 2 vs 240 in 5) 11.7 vs 12.7 us. Where
    // the wide grid is larger in few splits it wins: M=512 N=3072 K=12288 (384
    // vs 192 workgroups) 62.0 -> 47.3 us, M=128 N=K=5120 (160 vs 240 in 3
    // splits) 18.6 -> 15.7 us, M=48 N=9728 K=7488 (152 vs 228) 24.7 -> 20.5 us,
    // M=77 N=6448 K=10048 (202 vs 204 in 2) 28.4 -> 25.4 us (M=40 N=5552
    // K=6976, 174 vs 220 in 5 splits, would gain 5%).
    int bn = bm == 32 ? 128 : 64;
    if (bm == 64) {
        const int64_t t64 = (M + 63) / 64 * ((N + 63) / 64), t128 = (M + 63) / 64 * ((N + 127) / 128);
        const int64_t g64 = t64 * splits(t64), g128 = t128 * splits(t128);
        const bool wide = (g64 > target ? g128 < g64 : g128 <= target && g128 > g64) && splits(t128) <= 4;
        if (wide) bn = 128;
    }
    const int64_t tiles = (M + bm - 1) / bm * ((N + bn - 1) / bn);
    const int64_t ks = splits(tiles);
    pl.kernel_id = bm == 32 ? kLdsSk32x128 : bn == 128 ? kLdsSk64x128 : kLdsSk64x64;
    pl.ksplit = static_cast<int>(ks);
    pl.tiles = static_cast<int>(tiles);
    pl.counter_bytes = ks > 1 ? kWorkspaceCounterBytes : 0;
    pl.stages = nk / ks >= 64 ? 6 : 5;
    pl.workspace_bytes = ks > 1 ? pl.counter_bytes + static_cast<size_t>(tiles) * ks * bm * bn * 4 : 0;
    return pl;
}

bool launch_lds_splitk(const MmArgs& p, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const int target = p.smallm_min_groups > 0 ? p.smallm_min_groups : 256;
    const SplitKPlan pl = lds_splitk_plan(p.M, p.N, p.K, target);
    if (pl.kernel_id == 0) return false;
    int ks = pl.ksplit;
    uint32_t* counters = nullptr;
    float* partials = nullptr;
    if (ks > 1 && (pl.workspace_bytes == 0 || workspace == nullptr || workspace_bytes < pl.workspace_bytes)) ks = 1;
    if (ks > 1) {
        counters = static_cast<uint32_t*>(workspace);
        partials = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + pl.counter_bytes);
    }
    const int stages = ks == pl.ksplit ? pl.stages : p.K / kBK >= 64 ? 6 : 5;
    return lds_pipe_env() == 0 && !p.a_bf16
               ? launch_lds_pipe<0>(pl.kernel_id, p, stream, ks, partials, counters)
               : launch_lds_pipe<1>(pl.kernel_id, p, stream, ks, partials, counters, stages);
}

}  // namespace feather

