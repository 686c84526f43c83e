// LoRA down-projection T = x . D^T for the fused unmerged-LoRA epilogue.
//
// The reference's side path (comfy_feather/lora.py:4-35) starts every patch
// with temp = F.linear(x, lora_A): x (M, K) times the (rank, K) down matrix,
// fp32 accumulation, rounded to x's dtype. With the patches stacked along the
// rank (R = sum of ranks, padded to a multiple of 32) this is one skinny GEMM
// whose cost is reading x once (M = 4096, K = 3072: 25 MB of activations
// against 1.6 GFLOP). The kernel is built for that regime:
//   * a workgroup owns 64 or 128 rows of x and 16 * RN ranks (at most 128)
//     and walks its K range in 64-wide stages; x rows and D rows (128 bytes
//     per stage) arrive by whole-cache-line LDS-DMA copies into a three- or
//     four-stage ring that always keeps all but one stage in flight (copies
//     past a split's end repeat its last stage, so every wait count is a
//     constant), so the weight-like D is fetched once per row block, not per wave;
//   * 4 or 8 waves in a (rows/32) x 2 grid: wave (wm, wn) owns 32 rows and
//     half of the rank tiles, so every operand fragment read from LDS feeds
//     two MFMAs (16x16x32 fp16/bf16, D as the first operand: lane (lr, lg)
//     accumulates T[row lr][ranks 4*lg .. 4*lg+3]);
//   * 128-row blocks once M gives about one per CU; below that 64-row blocks
//     with the K range split as follows;
//   * for small M the K range is also split across workgroups (about one
//     workgroup per CU in total): each split stores its fp32 partial tile in
//     a caller workspace and bumps the tile's arrival counter, and the split
//     that arrives last adds the partials in split order (deterministic),
//     rounds and stores T, and re-zeroes the counter -- the arrival protocol
//     of the split-K GEMM tiles (device-coherent (sc1) 16-byte partial stores
//     and loads, a vmcnt wait before the barrier that precedes the counter RMW);
//   * rows past M read the last row (results dropped); 8-element K chunks past
//     K are zeroed in registers on both operands.
#include "feather_common.h"
#include "featherops_amd.h"
#include "lds_dma.h"
#include "lora_down.h"
#include "scaled_mm_dispatch.h"

namespace feather {
namespace {

constexpr int kLdBK = 64;  // K per stage

// WM x WN waves; wave (wm, wn) owns rows 32 wm .. 32 wm + 31 (two 16-row tiles) and
// rank tiles wn * RN / WN .. of the workgroup's 32 * WM rows x 16 * RN ranks.
template <int WM, int WN, int RN, bool kBf16, int kStagesReq>
__global__ __launch_bounds__(64 * WM * WN) void lora_down_kernel(const uint16_t* __restrict__ x,
                                                                  const uint16_t* __restrict__ d,
                                                                  uint16_t* __restrict__ t, int M, int K, int R,
                                                                  int r_base, int ksplit, float* __restrict__ partials,
                                                                  uint32_t* __restrict__ counters) {
    constexpr int kWaves = WM * WN;
    constexpr int kRows = 32 * WM;
    constexpr int RNW = RN / WN;  // rank tiles per wave
    static_assert(RN % WN == 0, "rank tiles split evenly over the wave columns");
    constexpr int kXStage = kRows * 128;
    constexpr int kDStage = RN * 16 * 128;
    constexpr int kStage = kXStage + kDStage;
    constexpr int kXInst = kXStage / 1024;
    constexpr int kDInst = kDStage / 1024;
    static_assert(kXInst % kWaves == 0, "x copies split evenly over the waves");
    constexpr int kXPerWave = kXInst / kWaves;
    constexpr int kDPerWave = (kDInst + kWaves - 1) / kWaves;  // surplus slots repeat the last copy
    constexpr int kLoads = kXPerWave + kDPerWave;
    // stage ring: kStagesReq buffers where they fit in 150 KB of LDS, else as many as fit
    constexpr int kS = kStagesReq * kStage <= 150 * 1024 ? kStagesReq : 150 * 1024 / kStage;
    static_assert(kS >= 3, "at least a three-stage ring");
    __shared__ __attribute__((aligned(1024))) uint8_t sbuf[kS][kStage];

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int lr = lane & 15;
    const int lg = lane >> 4;
    // workgroup -> (tile, split): the splits of a tile are consecutive
    const int q = blockIdx.x % ksplit;
    const int rowblk = blockIdx.x / ksplit;
    const int m0 = rowblk * kRows;
    const int wm = wave % WM;
    const int wn = wave / WM;
    const int r0 = r_base + blockIdx.y * (16 * RN);
    const int tile = rowblk * gridDim.y + blockIdx.y;
    const int nst_all = (K + kLdBK - 1) / kLdBK;
    const int per = (nst_all + ksplit - 1) / ksplit;
    const int st0 = q * per;
    const int nst = (nst_all - st0) < per ? (nst_all - st0) : per;

    // copy i of this wave: x rows (i < kXPerWave) or D rows, 8 rows of 128 bytes
    // (chunk p of LDS row r holds logical chunk p ^ swz(r)). The global address is a
    // wave-uniform base (the tile's first x row / first D row) plus a per-lane
    // 32-bit offset: row offset + stage offset + chunk offset.
    const uint8_t* xbase = reinterpret_cast<const uint8_t*>(x) + static_cast<int64_t>(m0) * K * 2;
    const uint8_t* dbase = reinterpret_cast<const uint8_t*>(d) + static_cast<int64_t>(r0) * K * 2;
    uint32_t rowoff[kLoads];
    uint32_t coff[kLoads];
    uint32_t ldst[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        const bool is_x = i < kXPerWave;
        const int jd = (i - kXPerWave) * kWaves + wave;
        const int j = is_x ? i * kWaves + wave : (jd < kDInst ? jd : kDInst - 1);  // surplus slots repeat
        const int row = j * 8 + (lane >> 3);
        const int lrow = is_x ? (m0 + row < M ? m0 + row : M - 1) - m0 : row;
        rowoff[i] = static_cast<uint32_t>(lrow) * static_cast<uint32_t>(K) * 2u;
        coff[i] = static_cast<uint32_t>(((lane & 7) ^ swz(row)) * 16);
        ldst[i] = (is_x ? 0 : kXStage) + j * 1024;
    }
    // a chunk past K re-reads chunk 0 of its stage (in bounds); the operand
    // reads zero it
    auto issue_stage = [&](int b, int st) {
        const uint32_t kb = static_cast<uint32_t>((st0 + st) * kLdBK * 2);
        const uint32_t lb = lds_addr_of(sbuf[b]);
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const uint32_t o = rowoff[i] + kb + (kb + coff[i] < static_cast<uint32_t>(K) * 2u ? coff[i] : 0u);
            dma16_lds(i < kXPerWave ? xbase : dbase, o, lb + ldst[i]);
        }
    };

    f32x4 acc[2][RNW];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int rn = 0; rn < RNW; ++rn) acc[i][rn] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto lds_ld16 = [](uint32_t addr) -> uint4 {
        using v4 = uint32_t __attribute__((ext_vector_type(4)));
        const v4 v = *reinterpret_cast<const __attribute__((address_space(3))) v4*>(static_cast<uintptr_t>(addr));
        return make_uint4(v.x, v.y, v.z, v.w);
    };
    auto compute = [&](int b, int st) {
        const uint32_t lb = lds_addr_of(sbuf[b]);
        const int kbase = (st0 + st) * kLdBK;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            // lane group lg holds logical chunk 2 * lg + h of every row
            const int ch = 2 * lg + h;
            const bool live = kbase + ch * 8 < K;
            uint4 xa[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int xr = wm * 32 + i * 16 + lr;
                xa[i] = lds_ld16(lb + xr * 128 + ((ch ^ swz(xr)) << 4));
                if (!live) xa[i] = make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int rn = 0; rn < RNW; ++rn) {
                const int dr = (wn * RNW + rn) * 16 + lr;
                uint4 db = lds_ld16(lb + kXStage + dr * 128 + ((ch ^ swz(dr)) << 4));
                if (!live) db = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    if constexpr (kBf16) acc[i][rn] = mfma16x16x32_bf16(db, xa[i], acc[i][rn]);
                    else acc[i][rn] = mfma16x16x32(as_half8(db), as_half8(xa[i]), acc[i][rn]);
                }
            }
        }
    };

    // kS-stage ring: copies of stages st + 1 .. st + kS - 2 in flight while st is
    // multiplied. kS - 1 stages are always in flight: a stage past the split's end
    // copies its last stage again into a buffer nothing reads, so every wait count
    // is a constant. (The planner gives every split at least one stage; the guard
    // keeps an empty split's copies from reading past the ends of x and D regardless.)
    if (nst > 0) {
#pragma unroll
        for (int i = 0; i < kS - 1; ++i) issue_stage(i, i < nst ? i : nst - 1);
    }
    for (int st = 0; st < nst; ++st) {
        wait_vmcnt<(kS - 2) * kLoads>();
        stage_barrier();  // stage st landed for every wave; stage st - 1's buffer is free
        const int nx = st + kS - 1;
        issue_stage(nx % kS, nx < nst ? nx : nst - 1);
        compute(st % kS, st);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): reads of this buffer done before it is refilled
    }
    wait_vmcnt<0>();  // the repeated copies past the end

    if (ksplit > 1) {
        // partial tile in fragment order ([wave][rn][lane], 16 bytes each) through
        // device-coherent (sc1) 16-byte buffer accesses, acknowledged (vmcnt) before
        // the barrier that precedes the arrival count
        constexpr int kTileBytes = kRows * RN * 16 * 4;
        constexpr int kCoherent = 16;  // sc1
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            partials + static_cast<int64_t>(tile) * ksplit * (kTileBytes / 4), 0, ksplit * kTileBytes, 0x00020000);
        auto frag = [&](int i, int rn) { return (((wave * 2 + i) * RNW + rn) * 64 + lane) * 16; };
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int rn = 0; rn < RNW; ++rn)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][rn]), prs,
                                                       q * kTileBytes + frag(i, rn), 0, kCoherent);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __shared__ int last_flag;
        __syncthreads();
        if (tid == 0)
            last_flag = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                        static_cast<uint32_t>(ksplit - 1);
        __syncthreads();
        if (!last_flag) return;
        // the splits are added in split order, kQ splits' loads in flight at a time
        constexpr int kQ = RNW <= 1 ? 4 : RNW <= 2 ? 2 : 1;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int rn = 0; rn < RNW; ++rn) acc[i][rn] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int q0 = 0; q0 < ksplit; q0 += kQ) {
            f32x4 p[kQ][2][RNW];
#pragma unroll
            for (int j = 0; j < kQ; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int rn = 0; rn < RNW; ++rn)
                        p[j][i][rn] = q0 + j < ksplit
                                          ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                          prs, (q0 + j) * kTileBytes + frag(i, rn), 0,
                                                                          kCoherent))
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < kQ; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int rn = 0; rn < RNW; ++rn) acc[i][rn] += p[j][i][rn];
        }
        if (tid == 0)  // ready for the next call on this stream
            __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int m = m0 + wm * 32 + i * 16 + lr;
        if (m < M) {
#pragma unroll
            for (int rn = 0; rn < RNW; ++rn) {
                const int r = r0 + (wn * RNW + rn) * 16 + 4 * lg;
                const uint2 o = make_uint2(f32x2_to_out_bits<kBf16>(acc[i][rn][0], acc[i][rn][1]),
                                           f32x2_to_out_bits<kBf16>(acc[i][rn][2], acc[i][rn][3]));
                *reinterpret_cast<uint2*>(t + static_cast<int64_t>(m) * R + r) = o;
            }
        }
    }
}

// The launches of one call: rank chunks of 128 (RN = 8) and one remainder chunk.
struct LoraChunk {
    int r_base, rn, nchunks;
};

int lora_chunks(int64_t R, LoraChunk out[2]) {
    int n = 0;
    const int full = static_cast<int>(R / 128);
    const int rest = static_cast<int>(R % 128);
    if (full > 0) out[n++] = LoraChunk{0, 8, full};
    if (rest > 0) out[n++] = LoraChunk{full * 128, rest / 16, 1};
    return n;
}

// Row block: 128 rows (8 waves) once M gives about one such workgroup per CU,
// else 64 rows (4 waves) with K split across workgroups.
int lora_rows(int64_t M, int nchunks) { return (M + 127) / 128 * nchunks >= 224 ? 128 : 64; }

// K split for this launch: as many splits as keep the grid within one
// workgroup per CU (at most 16, at least two stages per split). Rounding the
// split count down rather than up: M=4608 K=3072 R=64 (72 row blocks, 216 vs
// 288 workgroups) 2435 vs 2315 GB/s on the four-stage ring.
int lora_ksplit(int64_t M, int64_t K, int nchunks) {
    const int rows = lora_rows(M, nchunks);
    const int64_t tiles = (M + rows - 1) / rows * nchunks;
    const int64_t nst = (K + kLdBK - 1) / kLdBK;
    if (tiles > kWorkspaceCounters) return 1;
    int64_t ks = 256 / tiles;
    if (ks > nst / 2) ks = nst / 2;
    if (ks > 16) ks = 16;
    if (ks <= 1) return 1;
    // the kernel gives split q the stages [q * per, min((q + 1) * per, nst)):
    // drop trailing splits that would own none (K = 4160: 65 stages, 16 splits
    // of 5 cover them with 13)
    const int64_t per = (nst + ks - 1) / ks;
    ks = (nst + per - 1) / per;
    return static_cast<int>(ks);
}

size_t chunk_workspace(int64_t M, int64_t K, const LoraChunk& c) {
    const int ks = lora_ksplit(M, K, c.nchunks);
    if (ks <= 1) return 0;
    const int rows = lora_rows(M, c.nchunks);
    const int64_t tiles = (M + rows - 1) / rows * c.nchunks;
    return kWorkspaceCounterBytes + static_cast<size_t>(tiles) * ks * rows * c.rn * 16 * 4;
}

template <int WM, int RN>
void launch_wm(const LoraDownArgs& a, const LoraChunk& c, int ks, float* partials, uint32_t* counters,
               hipStream_t stream) {
    constexpr int kRows = 32 * WM;
    const dim3 grid(static_cast<uint32_t>((a.M + kRows - 1) / kRows * ks), static_cast<uint32_t>(c.nchunks));
    const dim3 block(64 * WM * 2);
    // stage ring: four stages for chunks of up to 64 ranks, three above (GB/s on x + D + T,
    // back to back, bf16, against the three-stage loop with branches around its tail
    // copies and a full wait at the tail: M=4096 K=3072 R=32 / 64 / 128 2931 / 2377 / 1834
    // vs 2763 / 2226 / 1748 (four stages at R=128: 1663); M=4096 K=12288 R=64 3995 vs 3501;
    // M=4096 K=5120 R=256 1612 vs 1407; M=32768 K=5120 R=64 5440 vs 5412; five and six
    // stages measured slower on these shapes; at one to four row blocks every form is within
    // 2% and the earlier loop slightly ahead (M=16 K=3072 R=64: 54.4 vs 55.4 GB/s)
    constexpr int kS = RN <= 4 ? 4 : 3;
    if (a.bf16)
        hipLaunchKernelGGL((lora_down_kernel<WM, 2, RN, true, kS>), grid, block, 0, stream, a.x, a.d, a.t,
                           static_cast<int>(a.M), static_cast<int>(a.K), static_cast<int>(a.R), c.r_base, ks, partials,
                           counters);
    else
        hipLaunchKernelGGL((lora_down_kernel<WM, 2, RN, false, kS>), grid, block, 0, stream, a.x, a.d, a.t,
                           static_cast<int>(a.M), static_cast<int>(a.K), static_cast<int>(a.R), c.r_base, ks, partials,
                           counters);
}

template <int RN>
void launch_rn(const LoraDownArgs& a, const LoraChunk& c, int ks, float* partials, uint32_t* counters,
               hipStream_t stream) {
    if (lora_rows(a.M, c.nchunks) == 128) launch_wm<4, RN>(a, c, ks, partials, counters, stream);
    else launch_wm<2, RN>(a, c, ks, partials, counters, stream);
}

}  // namespace

size_t lora_down_workspace_bytes(int64_t M, int64_t K, int64_t R) {
    LoraChunk cs[2];
    const int n = lora_chunks(R, cs);
    size_t need = 0;
    for (int i = 0; i < n; ++i) {
        const size_t w = chunk_workspace(M, K, cs[i]);
        if (w > need) need = w;
    }
    return need;
}

void launch_lora_down(const LoraDownArgs& a, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    LoraChunk cs[2];
    const int n = lora_chunks(a.R, cs);
    for (int i = 0; i < n; ++i) {
        const LoraChunk& c = cs[i];
        int ks = lora_ksplit(a.M, a.K, c.nchunks);
        const size_t need = chunk_workspace(a.M, a.K, c);
        if (ks > 1 && (workspace == nullptr || workspace_bytes < need)) ks = 1;  // no room: unsplit
        uint32_t* counters = ks > 1 ? static_cast<uint32_t*>(workspace) : nullptr;
        float* partials =
            ks > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + kWorkspaceCounterBytes) : nullptr;
        switch (c.rn) {
            case 2: launch_rn<2>(a, c, ks, partials, counters, stream); break;
            case 4: launch_rn<4>(a, c, ks, partials, counters, stream); break;
            case 6: launch_rn<6>(a, c, ks, partials, counters, stream); break;
            default: launch_rn<8>(a, c, ks, partials, counters, stream); break;
        }
    }
}

}  // namespace feather
