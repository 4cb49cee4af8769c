// gemm_mfma.hip -- the prefill GEMMs written for gfx950: y[m][n] (+)= x[m][k]
// . W[n][k]^T with bf16 operands and fp32 accumulation on
// v_mfma_f32_16x16x32_bf16.  The counterpart of the reference's prefill GEMM
// shaders (pf_gemm_t32.comp, dispatched at VulkanBackend.cs:782-856): W is a
// layer's bf16 dense copy (features x k), x the prompt rows (tokens x k).
//
// Workgroup tile: TF = 32 IF features x TT = 32 JT tokens, 4 waves of
// (TF / 2) x (TT / 2) (2 x 2), so a wave runs IF x JT MFMAs per 32-k step from
// IF + JT operand fragments.  The tile sizes are template arguments
// (128 x 128, 256 x 128, 128 x 256, 192 x 128, 192 x 256): a tile of TF x TT reads
// (TF + TT) / (TF TT) operand bytes per flop from L2, and the rate at which a
// CU receives operand rows is what bounds these GEMMs (below), so larger tiles
// are faster wherever there are enough of them to fill the chip.
//
// k advances in stages of 64: a stage is (TF + TT) / 16 row blocks of 2 KiB
// (16 rows x 64 k; the W blocks first, then the x blocks), copied from global
// memory straight into an LDS ring of S stages (global_load_lds_dwordx4).
// Each copy instruction reads 8 whole 128-byte lines (8 rows x 64 k); the
// rows' order and an XOR order of each row's 16-byte pieces place them in LDS
// so that the operand reads are free of bank conflicts.  The copy pattern sets the
// operand rate: on the o projection (2048^3) the 128 x 128 kernel took 36 us
// with each instruction reading 16 rows x 64 bytes (the same half of 16
// lines), 29 us with the halves alternating by row, and 25 us with whole
// lines, with identical output bits.
//
// The operands of one 32-k step are read from LDS into registers while the
// MFMAs of the previous step run.  Between
// the two steps of a stage the waves meet at a barrier once the next stage's
// copies have landed, and refill a free slot of the ring.
//
// Split k (SPLIT = 2, for outputs too small to give every CU a large tile):
// the two workgroups of a tile take the two halves of k.  The first to finish
// (a device-scope ticket per tile) stores its fp32 partial with
// device-coherent stores and marks it ready; the second adds it to its own
// with one fp32 addition per element, which is commutative, so the bits do
// not depend on which half finished first, and writes the tile.  The second
// waits only for a workgroup that is already running its stores, and that
// wait is bounded: past the bound the tile is written as NaN.
//
// Output: MFMA row = feature, column = token, so lane (grp, c) holds features
// 4 grp .. 4 grp + 3 of token c: one 16-byte store per 16 x 16 block (8 for
// bf16).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>

#include "device_common.hpp"
#include "ktimer.hpp"
#include "weights.hpp"

namespace hymt {
namespace {

constexpr int kBK = 64;               // k per stage
constexpr int kFrag = 1024;           // bytes of one 16 x 32 operand fragment
constexpr int kPair = 2 * kFrag;      // one row block's 16 rows x 64 k of a stage
constexpr int kGroupF = 4;            // feature tiles walked together (L2 reuse)
constexpr unsigned kSpinLimit = 1u << 22;  // polls of a split tile's ready mark

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct GemmArgs {
    const uint16_t *W;  // [n][k]; GLU: the gate rows [n / 2][k]
    const uint16_t *W2; // GLU: the up rows [n / 2][k]
    const uint16_t *x;  // [m][k]
    void *y;            // [m][ldy], fp32 or bf16
    int n, k, m, ldy;
    int tiles_f, tiles_t, group_f;
    int xcd_per;        // workgroups per XCD run, 0: identity order
    int kt;             // stages per workgroup (k / SPLIT / 64)
    float *part;        // SPLIT: partial tiles [tile][TF TT] in lane order
    unsigned *ticket;   // SPLIT: one per tile, 32 words apart, zero between calls
};

// s_waitcnt with vmcnt (<= 63) constrained and lgkmcnt left at its "no wait"
// maximum, or (the _L form) waited to zero too (gfx9 encoding: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
#define HYMT_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
#define HYMT_WAIT_VM_L(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const void *base) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, 0x7fffffff, 0x00020000);
}
constexpr int kSc1 = 16;  // buffer cache policy: device-coherent (sc1)

// Workgroup b runs on XCD b % 8 (dispatch is round-robin over the 8 XCDs).
// Tile order: groups of group_f feature tiles, walked token tile by token
// tile, so that the workgroups an XCD holds at a time share their W and x
// rows in that XCD's L2; each XCD takes one contiguous run of that order (of
// workgroups: the two k halves of a split tile are neighbours).
template <int SPLIT>
__device__ __forceinline__ void tile_of(const GemmArgs &a, int b, int &tile, int &tf, int &tt, int &kz) {
    const int L = a.xcd_per ? (b & 7) * a.xcd_per + (b >> 3) : b;
    tile = L / SPLIT;
    kz = L - tile * SPLIT;
    const int per_group = a.group_f * a.tiles_t;
    const int g = tile / per_group, r = tile - g * per_group;
    tt = r / a.group_f;
    tf = g * a.group_f + (r - tt * a.group_f);
}

// The schedule of a step, row by row: row i's JT MFMAs, then its reads (W
// fragment i and the x fragments the row loads).
template <int IF, int JT, int I>
__device__ __forceinline__ void sched_rows() {
    if constexpr (I < IF) {
        __builtin_amdgcn_sched_group_barrier(0x008, JT, 0);                                   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1 + (I + 1) * JT / IF - I * JT / IF, 0);  // DS read
        sched_rows<IF, JT, I + 1>();
    }
}

// One 32-k step of a wave: the IF x JT MFMAs of the operands in (w, cx),
// row by row, with the operand reads of the next step (LDS at nsb + noff,
// this lane's bytes) interleaved: W fragment i of the next step replaces w[i]
// as soon as row i's MFMAs have issued, and the x fragments go to nx, so a
// wave holds IF + 2 JT fragments.  after_row(i) runs after row i's reads
// (the stage copies spread over the step).
template <int IF, int JT, typename F>
__device__ __forceinline__ void substep(bf16x8 (&w)[IF], const bf16x8 (&cx)[JT], const uint8_t *nsb,
                                        uint32_t noff, int wf, int wt, bf16x8 (&nx)[JT], f32x4 (&acc)[IF][JT],
                                        F &&after_row) {
    constexpr int NBF = 2 * IF;  // W row blocks of a stage
#pragma unroll
    for (int i = 0; i < IF; i++) {
#pragma unroll
        for (int j = 0; j < JT; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[i], cx[j], acc[i][j], 0, 0, 0);
        w[i] = *(const bf16x8 *)(nsb + noff + (IF * wf + i) * kPair);
#pragma unroll
        for (int j = i * JT / IF; j < (i + 1) * JT / IF; j++)
            nx[j] = *(const bf16x8 *)(nsb + noff + (NBF + JT * wt + j) * kPair);
        after_row(i);
    }
    sched_rows<IF, JT, 0>();
}

// The MFMAs of a tile over the workgroup's k range by 2 x WT waves: wave
// (wf, wt) takes the tile's feature half wf and token part wt, IF x BJ
// 16 x 16 blocks (WT = 2: one wave per SIMD; WT = 4: two, each with half the
// accumulators, for tiles whose 4-wave accumulators and operands would not
// fit a wave's 256 VGPRs).  S stages in the LDS ring; LGKM: a stage's slot is
// refilled at the barrier right after its last operand reads (each wave first
// waits for its own reads: lgkmcnt(0)), so S - 1 stages are ahead of the one
// being read; else one barrier later, with S - 2 stages ahead and no wait on
// the reads.
//
// GLU (the gate/up GEMM with SwiGLU fused, unsplit): the tile's first TF / 2
// features are gate rows f0 / 2 + [0, TF / 2) of W, the others the same rows
// of W2 (up), so the tile holds both inputs of TF / 2 outputs
// silu(g) u (swiglu8, the row kernel's function of the same bf16-rounded g
// and u), written to y[m][ldy] at column f0 / 2: n is twice the output width.
template <int IF, int JT, int WT, int S, bool LGKM, int SPLIT, bool YBF16, bool ACC, bool GLU = false>
__global__ __launch_bounds__(128 * WT, 1) void gemm_kernel(GemmArgs a) {
    constexpr int TF = 32 * IF, TT = 32 * JT;
    constexpr int NW = 2 * WT, NT = 64 * NW, BJ = TT / (16 * WT);  // waves, threads, token blocks per wave
    constexpr int NBF = TF / 16, NB = (TF + TT) / 16;               // row blocks: W, all
    constexpr int C = 2 * NB / NW;                                   // copy instructions per wave per stage
    constexpr int kStageBytes = NB * kPair;
    constexpr int AHEAD = LGKM ? S : S - 1;  // stages issued ahead of the one being read, plus one
    static_assert((2 * NB) % NW == 0 && BJ >= 1 && AHEAD >= 2 && C * (AHEAD - 1) <= 63, "tile shape");
    static_assert(S * kStageBytes <= 160 * 1024, "LDS");
    static_assert(!GLU || (YBF16 && SPLIT == 1), "GLU: bf16 output, unsplit");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S * kStageBytes];
    unsigned &s_role = *(unsigned *)lds;  // split role, once the ring is idle
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = lane >> 4, c = lane & 15;
    int tile, tf, tt, kz;
    tile_of<SPLIT>(a, blockIdx.x, tile, tf, tt, kz);
    const int f0 = tf * TF, t0 = tt * TT;
    const int kt = a.kt;
    const size_t kbase = (size_t)kz * kt * kBK;

    // Staging: wave w issues loads g = C w + [0, C) of a stage, load g the
    // half h = g & 1 of row block gb = g >> 1 (W blocks first, then x): a
    // block's 2 KiB in two loads, each of 8 whole rows.
    // The block's 16 slot groups of 128 bytes hold its rows in the order
    // 0, 8, 1, 9, ..., 7, 15: group a = 8 h + (l >> 3) of load h holds row
    // (a >> 1) + 8 (a & 1), lane l taking that row's 16-byte piece
    // (l & 7) ^ (a >> 1) and landing in LDS slot l of the block's half h.
    // Each load reads 8 whole 128-byte lines.  Row c of a block (i = c >> 3,
    // r = c & 7) thus keeps piece p in slot 16 r + 8 i + (p ^ r); see the
    // operand offsets below.
    uint32_t voff[C];
    const uint16_t *sbase[C];
#pragma unroll
    for (int j = 0; j < C; j++) {
        const int g = wave * C + j, gb = g >> 1, h = g & 1;
        const int ga = 8 * h + (lane >> 3);
        const int rl = (ga >> 1) + 8 * (ga & 1);
        const int piece = (lane & 7) ^ (ga >> 1);
        const bool isw = gb < NBF;
        if constexpr (GLU) {  // gate row blocks [0, NBF / 2), then up
            const bool up = isw && gb >= NBF / 2;
            const int row = isw ? f0 / 2 + 16 * (up ? gb - NBF / 2 : gb) + rl : min(t0 + 16 * (gb - NBF) + rl, a.m - 1);
            voff[j] = (uint32_t)(((size_t)row * a.k + 8 * piece) * 2);
            sbase[j] = (isw ? (up ? a.W2 : a.W) : a.x) + kbase;
        } else {
            const int row = isw ? f0 + 16 * gb + rl : min(t0 + 16 * (gb - NBF) + rl, a.m - 1);
            voff[j] = (uint32_t)(((size_t)row * a.k + 8 * piece) * 2);
            sbase[j] = (isw ? a.W : a.x) + kbase;
        }
    }
    const uint32_t lds0 = lds_addr(lds) + wave * C * kFrag;
    // copy j of stage t into its ring slot t % S.  Stages past the last
    // (t >= kt) copy the last stage's rows again: their slots are never read
    // (a stage t >= kt shares its slot only with stages >= kt, or, with LGKM,
    // with the one stage whose reads ended before the barrier it follows), and
    // every iteration then issues C copies, so every wait below is the
    // steady-state count and the loop has no branch.
    auto copy = [&](int t, int j) __attribute__((always_inline)) {
        lds_dma16_sv(sbase[j] + min(t, kt - 1) * kBK, voff[j], lds0 + (t % S) * kStageBytes + j * kFrag);
    };
    // A stage's copies are spread over the MFMA rows of two steps: copies
    // [0, CB) in the step after the barrier that frees its slot, [CB, C) in
    // the next one.  Issued back to back after the barrier, the 4 waves' C
    // copies each held their wave for about 50 cycles a copy (the copy path
    // taking about 12 cycles per 1 KiB copy of the CU), and the MFMAs
    // waited.
    // With two stages ahead (AHEAD = 2) the wait right after the next step
    // lands the stage, so all its copies go in the step after the barrier.
    constexpr int CB = AHEAD > 2 ? (C + 1) / 2 : C;
    auto first_half = [&](int t) __attribute__((always_inline)) {
        return [&, t](int i) __attribute__((always_inline)) {
#pragma unroll
            for (int j = i * CB / IF; j < (i + 1) * CB / IF; j++) copy(t, j);
        };
    };
    auto second_half = [&](int t) __attribute__((always_inline)) {
        return [&, t](int i) __attribute__((always_inline)) {
#pragma unroll
            for (int j = CB + i * (C - CB) / IF; j < CB + (i + 1) * (C - CB) / IF; j++) copy(t, j);
        };
    };
    auto no_copy = [](int) {};
    // Operand reads: lane (grp, c) takes row c, k 8 grp + [0, 8) of k step
    // ks, i.e. piece 4 ks + grp, at byte off[ks] of each row block.  A
    // 16-byte read of 16 lanes takes one LDS pass on gfx950 when lanes 0-7
    // fall in one 128-byte half of a 256-byte bank row and lanes 8-15 in the
    // other, each 8 on distinct 16-byte slots of their half: rows 0-7 sit in
    // even slot groups at slot p ^ r, rows 8-15 in odd ones
    // (SQ_LDS_BANK_CONFLICT reads 0; 4 cycles per read with rows in order).
    uint32_t off[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const int i = c >> 3, r = c & 7;
        off[ks] = 16 * (16 * r + 8 * i + ((4 * ks + grp) ^ r));
    }

    const int wf = wave & 1, wt = wave >> 1;
    f32x4 acc[IF][BJ];
#pragma unroll
    for (int i = 0; i < IF; i++)
#pragma unroll
        for (int j = 0; j < BJ; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // kt >= 2.  A wave's copies (C a stage) retire in order, so a wait for at
    // most C n outstanding copies lands all but the last n stages issued.
    // The prologue issues stages [0, AHEAD - 1) and the first half of stage
    // AHEAD - 1, whose second half the first step issues.
#pragma unroll
    for (int t = 0; t < AHEAD - 1; t++)
#pragma unroll
        for (int j = 0; j < C; j++) copy(t, j);
#pragma unroll
    for (int j = 0; j < CB; j++) copy(AHEAD - 1, j);
    HYMT_WAIT_VM(C * (AHEAD - 2) + CB);
    asm volatile("s_barrier" ::: "memory");
    bf16x8 w[IF], ax[BJ], bx[BJ];
#pragma unroll
    for (int i = 0; i < IF; i++) w[i] = *(const bf16x8 *)(lds + off[0] + (IF * wf + i) * kPair);
#pragma unroll
    for (int j = 0; j < BJ; j++) ax[j] = *(const bf16x8 *)(lds + off[0] + (NBF + BJ * wt + j) * kPair);

    // The last stage is peeled: with its branch inside the loop, the
    // accumulators of the two paths met at the loop's join and the compiler
    // staged every MFMA's accumulator input through one register quad (four
    // v_accvgpr_mov_b32 per MFMA, 60 a stage at 128 x 128).
    for (int s = 0; s < kt - 1; s++) {
        // step (s, 0): its operands in (w, ax); read step (s, 1) into (w, bx);
        // the second half of stage s - 1 + AHEAD
        substep<IF, BJ>(w, ax, lds + (s % S) * kStageBytes, off[1], wf, wt, bx, acc, second_half(s - 1 + AHEAD));
        // stage s + 1 landed: stages up to s - 1 + AHEAD are issued, and
        // AHEAD - 2 of them may stay in flight
        if constexpr (LGKM) HYMT_WAIT_VM_L(C * (AHEAD - 2));
        else HYMT_WAIT_VM(C * (AHEAD - 2));
        asm volatile("s_barrier" ::: "memory");
        // step (s, 1): operands in (w, bx); read step (s + 1, 0) into (w, ax);
        // the first half of stage s + AHEAD
        substep<IF, BJ>(w, bx, lds + ((s + 1) % S) * kStageBytes, off[0], wf, wt, ax, acc, first_half(s + AHEAD));
    }
    substep<IF, BJ>(w, ax, lds + ((kt - 1) % S) * kStageBytes, off[1], wf, wt, bx, acc, no_copy);
#pragma unroll
    for (int i = 0; i < IF; i++)
#pragma unroll
        for (int j = 0; j < BJ; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[i], bx[j], acc[i][j], 0, 0, 0);
    HYMT_WAIT_VM(0);  // the copies past the last stage have landed before the ring is reused or freed

    if constexpr (SPLIT == 2) {
        // Ticket values of a tile within one call: the first arrival takes
        // 0 -> 1 and, once its partial is stored, adds 2; the second arrival
        // reads 1 (partial pending) or 3 (stored) and sets 0 for the next call.
        unsigned *tk = a.ticket + (size_t)tile * 32;
        __syncthreads();  // every wave's operand reads are done: the ring is idle
        if (tid == 0) s_role = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        const unsigned role = s_role;
        const __amdgpu_buffer_rsrc_t pr = part_rsrc(a.part + (size_t)tile * TF * TT);
        if (role == 0) {
#pragma unroll
            for (int i = 0; i < IF; i++)
#pragma unroll
                for (int j = 0; j < BJ; j++) {
                    const f32x4 v = acc[i][j];
                    const u32x4 u = {__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                     __float_as_uint(v[3])};
                    __builtin_amdgcn_raw_buffer_store_b128(u, pr, ((i * BJ + j) * NT + tid) * 16, 0, kSc1);
                }
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(0);  // every store acknowledged
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __syncthreads();
            if (tid == 0) __hip_atomic_fetch_add(tk, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return;
        }
        if (tid == 0) {
            unsigned v = role, spins = 0;
            if (role == 1) {
                do {
                    __builtin_amdgcn_s_sleep(2);
                    v = __hip_atomic_load(tk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } while (v != 4u && ++spins < kSpinLimit);
                v = v == 4u ? 3u : 0u;
            }
            s_role = v;  // 3: the partial is stored; else the tile is written as NaN
            __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        const bool ok = s_role == 3u;
#pragma unroll
        for (int i = 0; i < IF; i++) {
            u32x4 p[BJ];
#pragma unroll
            for (int j = 0; j < BJ; j++)
                p[j] = __builtin_amdgcn_raw_buffer_load_b128(pr, ((i * BJ + j) * NT + tid) * 16, 0, kSc1);
#pragma unroll
            for (int j = 0; j < BJ; j++) {
                f32x4 v = acc[i][j];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = ok ? v[e] + __uint_as_float(p[j][e]) : __builtin_nanf("");
                acc[i][j] = v;
            }
        }
    }

    // bf16 output: restaged through the (idle) ring as [token][feature] rows,
    // then written as whole 128-byte lines, 16 bytes a lane.  Written from the
    // MFMA layout, each 8-byte store reached 16 token rows, 32 bytes of each,
    // and the stores cost gate/up at m = 2048 about 14 of its 93 us.
    if constexpr (YBF16) {
        if ((a.ldy & 7) == 0) {
            constexpr int RS = TF + 8;        // row stride in bf16 elements (16 bytes of padding)
            constexpr int CPR = TF / 8;       // 16-byte chunks of a token row
            constexpr int NQ = TT * CPR / NT;  // chunks per thread
            static_assert(TT * RS * 2 <= S * kStageBytes && (TT * CPR) % NT == 0, "restage");
            uint16_t *st = (uint16_t *)lds;
            __syncthreads();  // every wave's operand reads (and the split handshake) are done
#pragma unroll
            for (int j = 0; j < BJ; j++) {
                const int tl = (TT / WT) * wt + 16 * j + c;
#pragma unroll
                for (int i = 0; i < IF; i++) {
                    const f32x4 v = acc[i][j];
                    *(uint2 *)(st + tl * RS + (TF / 2) * wf + 16 * i + 4 * grp) =
                        make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                                   (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
                }
            }
            __syncthreads();
            if constexpr (GLU) {
                constexpr int CPO = TF / 16;        // 16-byte chunks of an output row (TF / 2 values)
                constexpr int NO = TT * CPO / NT;   // chunks per thread
                static_assert((TT * CPO) % NT == 0, "GLU restage");
#pragma unroll
                for (int n = 0; n < NO; n++) {
                    const int q = n * NT + tid, row = q / CPO, col = q - row * CPO;
                    const int t = t0 + row;
                    if (t < a.m)
                        *(uint4 *)((uint16_t *)a.y + (size_t)t * a.ldy + f0 / 2 + 8 * col) =
                            swiglu8(*(const uint4 *)(st + row * RS + 8 * col),
                                    *(const uint4 *)(st + row * RS + TF / 2 + 8 * col));
                }
                return;
            }
#pragma unroll
            for (int n = 0; n < NQ; n++) {
                const int q = n * NT + tid, row = q / CPR, col = q - row * CPR;
                const int t = t0 + row;
                if (t < a.m)
                    *(uint4 *)((uint16_t *)a.y + (size_t)t * a.ldy + f0 + 8 * col) = *(const uint4 *)(st + row * RS + 8 * col);
            }
            return;
        }
    }

    // epilogue: lane (grp, c) of block (i, j) holds features f .. f + 3 of token t
#pragma unroll
    for (int j = 0; j < BJ; j++) {
        const int t = t0 + (TT / WT) * wt + 16 * j + c;
        if (t >= a.m) continue;
#pragma unroll
        for (int i = 0; i < IF; i++) {
            const int f = f0 + (TF / 2) * wf + 16 * i + 4 * grp;
            const f32x4 v = acc[i][j];
            if constexpr (YBF16) {
                uint16_t *yp = (uint16_t *)a.y + (size_t)t * a.ldy + f;
                *(uint2 *)yp = make_uint2((uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16),
                                          (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16));
            } else {
                float4 *yp = (float4 *)((float *)a.y + (size_t)t * a.ldy + f);
                float4 o = make_float4(v[0], v[1], v[2], v[3]);
                if constexpr (ACC) {
                    const float4 q = *yp;
                    o = make_float4(q.x + o.x, q.y + o.y, q.z + o.z, q.w + o.w);
                }
                *yp = o;
            }
        }
    }
}

// The tile shapes: IF, JT (features / 32, tokens / 32), ring depth, LGKM.
struct TileShape {
    const char *name;
    int IF, JT;
};
constexpr TileShape kTiles[kGemmTiles] = {
    {"128x128", 4, 4}, {"256x128", 8, 4}, {"128x256", 4, 8}, {"192x128", 6, 4}, {"192x256", 6, 8}, {"128x64", 4, 2},
    {"128x96", 4, 3}};

template <int IF, int JT, int WT, int S, bool LGKM, int SPLIT>
void launch_tile(const GemmArgs &a, int grid, bool y_bf16, bool acc, hipStream_t s, const KernelSpan &span,
                 bool glu = false) {
    const dim3 block(128 * WT);
    if constexpr (SPLIT == 1)
        if (glu) return launch(span, gemm_kernel<IF, JT, WT, S, LGKM, 1, true, false, true>, dim3(grid), block, 0, s, a);
    if (y_bf16) launch(span, gemm_kernel<IF, JT, WT, S, LGKM, SPLIT, true, false>, dim3(grid), block, 0, s, a);
    else if (acc) launch(span, gemm_kernel<IF, JT, WT, S, LGKM, SPLIT, false, true>, dim3(grid), block, 0, s, a);
    else launch(span, gemm_kernel<IF, JT, WT, S, LGKM, SPLIT, false, false>, dim3(grid), block, 0, s, a);
}

// Ring depths, measured at the model's shapes: deeper rings (128 x 128 with 5
// stages, 4 ahead) were no faster, so the stream is not latency-bound.
template <int SPLIT>
void launch_shape(int tile, const GemmArgs &a, int grid, bool y_bf16, bool acc, hipStream_t s,
                  const KernelSpan &span, bool glu = false) {
    switch (tile) {
    case 0: launch_tile<4, 4, 2, 4, false, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break;  // 32 KiB stages
    case 1: launch_tile<8, 4, 2, 3, true, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break;   // 48 KiB
    case 2: launch_tile<4, 8, 2, 3, true, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break;   // 48 KiB
    case 3: launch_tile<6, 4, 4, 4, true, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break;   // 40 KiB, 8 waves
    // 8 waves: 4 waves' 192 accumulators and operands each need more than
    // 256 VGPRs (the loop then moved accumulators through AGPRs); gate/up
    // at m = 2048 108 -> 94 us.  An 8-wave 256 x 256 tile took 105 us.  At
    // 192 x 128 8 waves gain 1-3 % (q/k/v at m = 2048, gate/up at 512); at
    // 128 x 128 they were mixed (down at m = 2048 2 % slower).
    case 4: launch_tile<6, 8, 4, 2, true, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break;   // 56 KiB
    // 128 x 64: short prompts, where 128 x 128 tiles leave a quarter of the
    // chip idle (at m = 512, split: o 11.4 against 15.0 us for 128 x 128 split,
    // down 22.9 against 28.1, q/k/v unsplit 13.3 against 15.3); a 192 x 64
    // tile was slower at every model shape
    case 5: launch_tile<4, 2, 2, 4, false, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break;  // 24 KiB
    default: launch_tile<4, 3, 2, 4, false, SPLIT>(a, grid, y_bf16, acc, s, span, glu); break; // 28 KiB
    }
}

int tiles_of(int tile, int n, int m) {
    const int TF = 32 * kTiles[tile].IF, TT = 32 * kTiles[tile].JT;
    if (n % TF) return 0;
    return (n / TF) * ((m + TT - 1) / TT);
}

// The share of its last round of workgroups a launch fills on 256 CUs
// (1: whole rounds).
double round_fill(int wgs) {
    if (wgs <= 0) return 0.0;
    const int rounds = (wgs + 255) / 256;
    return wgs / (256.0 * rounds);
}

}  // namespace

int gemm_tile_by_name(const char *name) {
    for (int t = 0; t < kGemmTiles; t++)
        if (!std::strcmp(name, kTiles[t].name)) return t;
    return -1;
}

// The tile plan for a shape: the tile whose workgroups fill whole rounds of
// the chip best, the larger tile on a tie, 192 rows where the width allows;
// with deep k (>= 4096) a k split of 128 x 128 tiles when they alone would
// fill less than three quarters of a round; else, for a short prompt, the
// k split of 128 x 64 tiles.  Measured (us per call, the plan's tile /
// hipBLASLt's first heuristic choice; `bench.py --only gemm`): at m = 2048
// q/k/v 192 x 128 27.2 / 28.1, gate/up 192 x 256 84.9 / 83.9, o 128 x 128
// 22.1 / 24.0, down 128 x 128 51.7 / 54.7; at m = 1531 q/k/v 192 x 128 21.5 /
// 22.8, gate/up 192 x 128 67.9 / 64.8, o and down 128 x 96 17.1 / 19.3 and
// 39.0 / 42.6; at m = 1024 q/k/v 128 x 128 17.6 / 18.6, gate/up 192 x 256
// 42.8 / 42.2, o 128 x 64 15.1 / 16.9, down 128 x 128 split 30.7 / 36.8; at
// m = 512 q/k/v 128 x 64 13.3 / 13.0, gate/up 192 x 128 27.4 / 28.2, o and
// down 128 x 64 split 11.4 / 11.6 and 22.9 / 26.6.
GemmPlan gemm_mfma_plan(int n, int k, int m) {
    // forced by HYMT_HIP_GEMM_TILE=<tile>[,2] (a tuning knob; the shape rules
    // still apply)
    if (const char *e = std::getenv("HYMT_HIP_GEMM_TILE")) {
        char buf[32];
        std::strncpy(buf, e, sizeof(buf) - 1);
        buf[sizeof(buf) - 1] = 0;
        char *comma = std::strchr(buf, ',');
        int split = 1;
        if (comma) {
            *comma = 0;
            split = std::atoi(comma + 1) == 2 ? 2 : 1;
        }
        const int t = gemm_tile_by_name(buf);
        if (t >= 0) return GemmPlan{t, split};
    }
    auto fill = [&](int t, int split) { return round_fill(tiles_of(t, n, m) * split); };
    if (n % 192 == 0) {
        const double e4 = fill(4, 1), e3 = fill(3, 1);
        if (std::max(e4, e3) >= 0.75) return GemmPlan{e4 >= e3 ? 4 : 3, 1};
    }
    int best = 0;  // 128 x 128, 128 x 96, 128 x 64: the best fill, the larger on a tie
    double eb = fill(0, 1);
    for (int t : {6, 5})
        if (fill(t, 1) > eb + 1e-9) {
            best = t;
            eb = fill(t, 1);
        }
    const bool splittable = k % 256 == 0;
    if (splittable && k >= 4096 && fill(0, 1) < 0.75 && fill(0, 2) >= 0.75) return GemmPlan{0, 2};
    if (eb >= 0.75 || !splittable) return GemmPlan{best, 1};
    return GemmPlan{5, 2};  // a short prompt
}

bool gemm_mfma_fits(const uint16_t *W, int n, int k, const uint16_t *x, int m, const void *y, int ldy) {
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    return n > 0 && n % 128 == 0 && k >= 2 * kBK && k % (2 * kBK) == 0 && m > 0 && ldy >= n && ldy % 4 == 0 &&
           (size_t)n * k * 2 < (1ull << 31) && (size_t)m * k * 2 < (1ull << 31) && a16(W) && a16(x) && a16(y);
}

size_t gemm_split_bytes(int n, int m, GemmPlan p) {
    if (p.split < 2) return 0;
    return (size_t)tiles_of(p.tile, n, m) * 32 * kTiles[p.tile].IF * 32 * kTiles[p.tile].JT * 4;
}

int gemm_split_tiles(int n, int m, GemmPlan p) {
    if (p.tile < 0 || p.tile >= kGemmTiles) return 0;
    const int t = tiles_of(p.tile, n, m);
    return t ? t : tiles_of(0, n, m);
}

hipError_t gemm_bf16_mfma(const uint16_t *W, int n, int k, const uint16_t *x, int m, void *y, int ldy, bool y_bf16,
                          bool accumulate, hipStream_t s, GemmPlan p, const GemmSplitWs *ws) {
    if (!gemm_mfma_fits(W, n, k, x, m, y, ldy) || (accumulate && y_bf16)) return hipErrorInvalidValue;
    if (p.tile < 0 || p.tile >= kGemmTiles) return hipErrorInvalidValue;
    int tiles = tiles_of(p.tile, n, m);
    if (!tiles) {  // n not a multiple of the tile's width
        p = GemmPlan{0, p.split};
        tiles = tiles_of(0, n, m);
    }
    // a split needs >= 2 stages per half and room for its partials and tickets
    if (p.split == 2 && (k % (4 * kBK) || !ws || ws->part_bytes < gemm_split_bytes(n, m, p) || ws->tickets < tiles))
        p.split = 1;
    const int TF = 32 * kTiles[p.tile].IF;
    GemmArgs a{};
    a.W = W;
    a.x = x;
    a.y = y;
    a.n = n;
    a.k = k;
    a.m = m;
    a.ldy = ldy;
    a.tiles_f = n / TF;
    a.tiles_t = tiles / a.tiles_f;
    a.group_f = a.tiles_f % kGroupF == 0 ? kGroupF : 1;
    a.kt = k / p.split / kBK;
    a.part = p.split == 2 ? (float *)ws->part : nullptr;
    a.ticket = p.split == 2 ? ws->ticket : nullptr;
    const int grid = tiles * p.split;
    a.xcd_per = grid % 8 == 0 ? grid / 8 : 0;
    KernelSpan span(y_bf16 ? "gemm_mfma_out_bf16" : "gemm_mfma_out_f32", s, true);
    if (p.split == 2) launch_shape<2>(p.tile, a, grid, y_bf16, accumulate, s, span);
    else launch_shape<1>(p.tile, a, grid, y_bf16, accumulate, s, span);
    return hipGetLastError();
}

bool gemm_swiglu_fits(const uint16_t *Wg, const uint16_t *Wu, int f, int k, const uint16_t *x, int m,
                      const uint16_t *act, int ld) {
    auto a16 = [](const void *p) { return ((uintptr_t)p & 15u) == 0; };
    return f > 0 && f % 64 == 0 && k >= 2 * kBK && k % (2 * kBK) == 0 && m > 0 && ld >= f && ld % 8 == 0 &&
           (size_t)f * k * 2 < (1ull << 31) && (size_t)m * k * 2 < (1ull << 31) && a16(Wg) && a16(Wu) && a16(x) &&
           a16(act);
}

hipError_t gemm_swiglu_mfma(const uint16_t *Wg, const uint16_t *Wu, int f, int k, const uint16_t *x, int m,
                            uint16_t *act, int ld, hipStream_t s, GemmPlan p) {
    if (!gemm_swiglu_fits(Wg, Wu, f, k, x, m, act, ld) || p.split != 1) return hipErrorInvalidValue;
    if (p.tile < 0 || p.tile >= kGemmTiles) return hipErrorInvalidValue;
    const int n = 2 * f;  // gate and up features, as the unfused GEMM sees them
    int tiles = tiles_of(p.tile, n, m);
    if (!tiles) {  // 2 f not a multiple of the tile's width (f % 64 == 0: 128 rows always fit)
        p.tile = 0;
        tiles = tiles_of(0, n, m);
    }
    const int TF = 32 * kTiles[p.tile].IF;
    GemmArgs a{};
    a.W = Wg;
    a.W2 = Wu;
    a.x = x;
    a.y = act;
    a.n = n;
    a.k = k;
    a.m = m;
    a.ldy = ld;
    a.tiles_f = n / TF;
    a.tiles_t = tiles / a.tiles_f;
    a.group_f = a.tiles_f % kGroupF == 0 ? kGroupF : 1;
    a.kt = k / kBK;
    a.xcd_per = tiles % 8 == 0 ? tiles / 8 : 0;
    KernelSpan span("gemm_mfma_swiglu", s, true);
    launch_shape<1>(p.tile, a, tiles, true, false, s, span, true);
    return hipGetLastError();
}

}  // namespace hymt
