// gemm_mfma.hip -- the prefill GEMMs written for gfx950: y[m][n] (+)= x[m][k]
// . W[n][k]^T with bf16 operands and fp32 accumulation on
// v_mfma_f32_16x16x32_bf16.  The counterpart of the reference's prefill GEMM
// shaders (pf_gemm_t32.comp, dispatched at VulkanBackend.cs:782-856): W is a
// layer's bf16 dense copy (features x k), x the prompt rows (tokens x k).
//
// Workgroup tile: 128 features x 128 tokens, 4 waves of 64 x 64 (2 x 2), so a
// wave runs 16 MFMAs per 32-k step from 8 operand fragments.  k advances in
// stages of 64; a stage is 16 row blocks of 2 KiB (16 rows x 64 k; 8 of W,
// 8 of x), copied from global memory straight into LDS
// (global_load_lds_dwordx4) four stages deep, so that three stages of loads
// are in flight behind the MFMAs.
//
// Each copy instruction reads 8 whole 128-byte lines (8 rows x 64 k), and
// its lanes take the 16-byte pieces of a row in an XOR order that places
// them in LDS so that the operand reads are conflict-free.  The copy pattern
// sets the operand rate: on the o projection (2048^3) the same kernel took
// 36 us with each instruction reading 16 rows x 64 bytes (the same half of
// 16 lines), 29 us with the halves alternating by row, and 25 us with whole
// lines, with identical output bits; padding the rows by 64 bytes had the
// alternating form's effect.  A tile alone on its CU streams its operand
// rows at about 21 bytes per clock this way, against 11 before.
//
// Output: MFMA row = feature, column = token, so lane (grp, c) holds features
// 4 grp .. 4 grp + 3 of token c: one 16-byte store per tile (8 for bf16).
//
// Measured on the MI355X at m = 2048, per call (with HYMT_HIP_GEMM=auto
// gemm.cpp times it against hipBLASLt's candidates on a shape's first call
// and keeps the faster): o 27.8-28.9 us against hipBLASLt's 26.4, down
// 68-75 against 58.9, so the library still serves the model's shapes; at
// m <= 1024 a shape has too few 128 x 128 tiles to fill the chip (16 at
// m = 128 for the o projection), where hipBLASLt splits k.  What bounds it,
// from timing-only variants of the o projection (2048^3, 25 us without
// accumulation): the operand stream.  Without the copies 15.7 us, without
// the LDS operand reads 23.7 (the reads hide under the MFMAs), without the
// output stores 20.6 (16 MB arriving as one wave of tiles ends; staging the
// output through LDS into whole-line stores did not change that).  In the
// steady state a 64-k stage takes about 1730 clocks with the copies and 750
// without, i.e. 32 KB per CU arrives at about 19 bytes per clock with every
// CU busy (25 with a tile alone on its CU), whether the ring holds 4 or 5
// stages or the copies go through registers (33 us, slower).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device_common.hpp"
#include "ktimer.hpp"
#include "weights.hpp"

namespace hymt {
namespace {

constexpr int kTF = 128;                  // features per workgroup
constexpr int kTT = 128;                  // tokens per workgroup
constexpr int kBK = 64;                   // k per stage
constexpr int kStages = 4;                // LDS ring depth (stages of kBK)
constexpr int kFrag = 1024;               // bytes of one 16 x 32 operand fragment
constexpr int kPair = 2 * kFrag;          // one row block's 16 rows x 64 k of a stage
constexpr int kStageBytes = 32 * kFrag;   // W row blocks 0..7, x row blocks 8..15
constexpr int kGroupF = 4;                // feature tiles walked together (L2 reuse)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint16_t *W;  // [n][k]
    const uint16_t *x;  // [m][k]
    void *y;            // [m][ldy], fp32 or bf16
    int n, k, m, ldy;
    int tiles_f, tiles_t, group_f;
    int xcd_per;        // tiles per XCD run, 0: identity order
};

// s_waitcnt with only vmcnt (<= 63) constrained (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt and lgkmcnt at their "no wait" maxima)
#define HYMT_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// Workgroup b runs on XCD b % 8 (dispatch is round-robin over the 8 XCDs).
// Tile order: groups of group_f feature tiles, walked token tile by token
// tile, so that the 32 workgroups an XCD holds at a time cover about 4 x 8
// tiles and share their W and x rows in that XCD's L2; each XCD takes one
// contiguous run of that order.
__device__ __forceinline__ void tile_of(const GemmArgs &a, int b, int &tf, int &tt) {
    const int L = a.xcd_per ? (b & 7) * a.xcd_per + (b >> 3) : b;
    const int per_group = a.group_f * a.tiles_t;
    const int g = L / per_group, r = L - g * per_group;
    tt = r / a.group_f;
    tf = g * a.group_f + (r - tt * a.group_f);
}

typedef bf16x8 Frags[2][4];  // [k step of 32][row block of 16]

// One stage of a wave: the 32 MFMAs of the operands in (cw, cx), with the 16
// operand reads of the next stage (LDS at sb, this lane's bytes) into (nw,
// nx) interleaved, one read per two MFMAs, so that the LDS and the matrix
// pipe work at the same time.
__device__ __forceinline__ void stage_step(const uint8_t *sb, const uint32_t (&off)[2], int wf, int wt,
                                           const Frags &cw, const Frags &cx, Frags &nw, Frags &nx,
                                           f32x4 (&acc)[4][4]) {
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            nw[ks][i] = *(const bf16x8 *)(sb + off[ks] + (4 * wf + i) * kPair);
            nx[ks][i] = *(const bf16x8 *)(sb + off[ks] + (8 + 4 * wt + i) * kPair);
        }
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cw[ks][i], cx[ks][j], acc[i][j], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; r++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // 2 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // 1 DS read
    }
}

template <bool YBF16, bool ACC, int STAGES>
__global__ __launch_bounds__(256, 1) void gemm_bf16_kernel(GemmArgs a) {
    static_assert(STAGES == 4, "the copy waits below count stages of a 4-slot ring");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[STAGES * kStageBytes];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, c = lane & 15;
    int tf, tt;
    tile_of(a, blockIdx.x, tf, tt);
    const int f0 = tf * kTF, t0 = tt * kTT;

    // Staging: wave w copies row blocks rb = 4 (w & 1) + [0, 4) of W (w < 2)
    // or of x (w >= 2), one block's 2 KiB in two loads, each of 8 whole
    // rows: load j takes rows 16 rb + 8 (j & 1) + [0, 8), lane l row l >> 3
    // and the 16-byte piece (l & 7) ^ (l >> 3) ^ (j & 1) of the row's
    // 128-byte stage.  Each load reads 8 whole 128-byte lines, and lands in
    // LDS slot l of the block's half j & 1.  Row c of a block (i = c >> 3,
    // r = c & 7) thus keeps piece p in slot 64 i + 8 r + (p ^ r ^ i); see
    // the operand offsets below.
    const bool stage_x = wave >= 2;
    const uint16_t *src[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        const int row = (wave & 1) * 64 + (j >> 1) * 16 + 8 * (j & 1) + (lane >> 3);
        const int piece = (lane & 7) ^ (lane >> 3) ^ (j & 1);
        src[j] = (stage_x ? a.x + (size_t)min(t0 + row, a.m - 1) * a.k : a.W + (size_t)(f0 + row) * a.k) + 8 * piece;
    }
    const uint32_t lds0 = lds_addr(lds) + wave * 8 * kFrag;
    auto issue = [&](int s) {
        const uint32_t dst = lds0 + (s % STAGES) * kStageBytes;
        const int kk = s * kBK;
#pragma unroll
        for (int j = 0; j < 8; j++) lds_dma16(src[j] + kk, dst + j * kFrag);
    };
    // Operand reads: lane (grp, c) takes row c, k 8 grp + [0, 8) of k step
    // ks, i.e. piece 4 ks + grp, at byte off[ks] of each row block.  The 16
    // lanes of one grp hit 16 distinct slots mod 16 (and any 8 consecutive
    // ones distinct slots mod 8), so the reads are free of bank conflicts.
    uint32_t off[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const int i = c >> 3, r = c & 7;
        off[ks] = 16 * (64 * i + 8 * r + ((4 * ks + grp) ^ r ^ i));
    }

    const int wf = wave & 1, wt = wave >> 1;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int kt = a.k / kBK;  // even, >= 2
#pragma unroll
    for (int s = 0; s < STAGES - 1; s++)
        if (s < kt) issue(s);
    // stage 0 into registers.  A wave's copies (8 a stage) retire in order,
    // so a wait for at most 8 n outstanding copies lands all but the last n
    // stages issued.  Each wait is one straight-line s_waitcnt: choosing the
    // count through a switch compiled to a branch tree that cost 5-10 % of
    // the kernel (o projection 24.9 -> 23.6 us, identical output bits).
    if (kt > 2) HYMT_WAIT_VM(16);
    else HYMT_WAIT_VM(8);
    asm volatile("s_barrier" ::: "memory");
    Frags aw, ax, bw, bx;
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            aw[ks][i] = *(const bf16x8 *)(lds + off[ks] + (4 * wf + i) * kPair);
            ax[ks][i] = *(const bf16x8 *)(lds + off[ks] + (8 + 4 * wt + i) * kPair);
        }
    // Stage s: its operands are in registers; make stage s + 1 visible (this
    // wave's copies landed, then a barrier for every wave's, which also
    // frees the slot of stage s - 1), refill that slot with stage
    // s + STAGES - 1, then the MFMAs of s with the reads of s + 1.  After the
    // last stage the reads fetch a stale slot, unused.
    auto step = [&](int s, const Frags &cw, const Frags &cx, Frags &nw, Frags &nx) {
        if (s + 1 < kt) {
            // stage s + 2 may stay in flight, none at the last refill
            if (s + 2 < kt) HYMT_WAIT_VM(8);
            else HYMT_WAIT_VM(0);
            asm volatile("s_barrier" ::: "memory");
            if (s + STAGES - 1 < kt) issue(s + STAGES - 1);
        }
        stage_step(lds + ((s + 1) % STAGES) * kStageBytes, off, wf, wt, cw, cx, nw, nx, acc);
    };
    for (int s = 0; s < kt; s += 2) {
        step(s, aw, ax, bw, bx);
        step(s + 1, bw, bx, aw, ax);
    }

    // epilogue: lane (grp, c) of tile (i, j) holds features f .. f + 3 of token t
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int t = t0 + 64 * wt + 16 * j + c;
        if (t >= a.m) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int f = f0 + 64 * wf + 16 * i + 4 * grp;
            const f32x4 v = acc[i][j];
            if constexpr (YBF16) {
                uint16_t *yp = (uint16_t *)a.y + (size_t)t * a.ldy + f;
                *(uint2 *)yp = make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                                          (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
            } else {
                float4 *yp = (float4 *)((float *)a.y + (size_t)t * a.ldy + f);
                float4 o = make_float4(v[0], v[1], v[2], v[3]);
                if constexpr (ACC) {
                    const float4 p = *yp;
                    o = make_float4(p.x + o.x, p.y + o.y, p.z + o.z, p.w + o.w);
                }
                *yp = o;
            }
        }
    }
}

}  // namespace

bool gemm_mfma_fits(const uint16_t *W, int n, int k, const uint16_t *x, int m, const void *y, int ldy) {
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    return n > 0 && n % kTF == 0 && k >= 2 * kBK && k % (2 * kBK) == 0 && m > 0 && ldy >= n && ldy % 4 == 0 && a16(W) &&
           a16(x) && a16(y);
}

hipError_t gemm_bf16_mfma(const uint16_t *W, int n, int k, const uint16_t *x, int m, void *y, int ldy, bool y_bf16,
                          bool accumulate, hipStream_t s) {
    if (!gemm_mfma_fits(W, n, k, x, m, y, ldy) || (accumulate && y_bf16)) return hipErrorInvalidValue;
    GemmArgs a;
    a.W = W;
    a.x = x;
    a.y = y;
    a.n = n;
    a.k = k;
    a.m = m;
    a.ldy = ldy;
    a.tiles_f = n / kTF;
    a.tiles_t = (m + kTT - 1) / kTT;
    a.group_f = a.tiles_f % kGroupF == 0 ? kGroupF : 1;
    const int tiles = a.tiles_f * a.tiles_t;
    a.xcd_per = tiles % 8 == 0 ? tiles / 8 : 0;
    KernelSpan span(y_bf16 ? "gemm_mfma_out_bf16" : "gemm_mfma_out_f32", s, true);
    if (y_bf16) launch(span, gemm_bf16_kernel<true, false, kStages>, dim3(tiles), dim3(256), 0, s, a);
    else if (accumulate) launch(span, gemm_bf16_kernel<false, true, kStages>, dim3(tiles), dim3(256), 0, s, a);
    else launch(span, gemm_bf16_kernel<false, false, kStages>, dim3(tiles), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace hymt
