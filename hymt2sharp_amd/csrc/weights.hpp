// weights.hpp -- device layout of the quantized weight matrices (decode GEMV).
//
// A matrix of rows x cols values arrives as rows of GGUF blocks (the bytes
// GgufFile hands to the reference's kernels; block structs in
// BlockLayout.cs:9-106).  hymt_weight_upload repacks it so that every 32-value
// unit of a row is read with aligned vector loads:
//   F32, F16   as stored, [rows][cols]
//   Q8_0       q: int8 [rows][cols]; d: fp32 [rows][cols/32]
//   Q4_K       q: the 144-byte super-blocks as stored (already 16-byte aligned)
//   Q6_K       q: 208-byte super-blocks ql[128] qh[64] scales[16]; d: fp32
//              [rows][cols/256]
//   Q2_0C      q: the code bytes [rows][cols/4]; d: fp32 [rows][cols/512]
//   STQ1_0     q: the slot bytes [rows][cols/8]; q2: the sign bytes
//              [rows][cols/32]; d: fp32 [rows][cols/256]
// (fp16 scales widened to fp32 exactly on the host).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <vector>

namespace hymt {

// GgmlTensorType codes (GgmlTensorType.cs)
constexpr int kW_F32 = 0, kW_F16 = 1, kW_Q8_0 = 8, kW_Q4_K = 12, kW_Q6_K = 14, kW_Q2_0C = 40, kW_STQ1_0 = 43;

struct WeightDev {
    int type, rows, cols;
    const void *q;
    const void *q2;
    const float *d;
};

// Bytes of one GGUF row of cols values; -1 for an unsupported type.
long gguf_row_bytes(int type, int cols);

// The device layout of a matrix: one buffer, q / q2 / d at 256-byte aligned
// offsets (q2, d = SIZE_MAX when absent).
struct PackedWeight {
    std::vector<uint8_t> buf;
    size_t off_q = 0, off_q2 = SIZE_MAX, off_d = SIZE_MAX;
};
bool pack_weight(int type, int rows, int cols, const uint8_t *src, PackedWeight &out);

// gemv flags (as HYMT_GEMV_* in include/hymt_hip.h)
constexpr int kGemvAccumulate = 1, kGemvInRmsNorm = 2, kGemvInSwiGLU = 4, kGemvOutSwiGLU = 8;
hipError_t launch_gemv(const WeightDev &w, const float *x, float *y, int flags, const float *nw, float eps,
                       hipStream_t s);
hipError_t launch_embed(const WeightDev &w, int row, float *out, hipStream_t s);
// n rows of W as fp32 rows at out: rows[i] (device array) or row0 + i
hipError_t launch_rows(const WeightDev &w, const int *rows, int row0, int n, float *out, hipStream_t s);
// row kernels of the prefill (rows.hip); bf16 outputs are RNE-rounded bits
hipError_t launch_rows_rmsnorm(const float *x, int m, int n, const float *w, float eps, uint16_t *out,
                               hipStream_t s);
hipError_t launch_rows_swiglu(const float *gu, int m, int n, uint16_t *out, hipStream_t s);
hipError_t launch_rows_swiglu_bf16(const uint16_t *gu, int m, int n, uint16_t *out, hipStream_t s);
hipError_t launch_to_bf16(const float *x, size_t count, uint16_t *out, hipStream_t s);
// y[m][n] (+)= x[m][k] . W[n][k]^T, bf16 operands, fp32 accumulation
// (gemm.cpp: this library's MFMA kernel, gemm_mfma.hip, wherever it fits,
// hipBLASLt's first heuristic choice elsewhere); y is fp32 or, with y_bf16,
// bf16, rows ldy elements apart.  The GemmState (library handle, workspace,
// chosen kernels) belongs to one context.  HYMT_HIP_GEMM, read when the state
// is created, changes the choice: =library hipBLASLt everywhere, =hipblaslt
// hipBLASLt's timed pick, =auto the faster of the two on the first call of a
// shape (=mfma is the default).
struct GemmState;
GemmState *gemm_state_create();
void gemm_state_destroy(GemmState *g);
hipError_t gemm_bf16(GemmState *g, hipStream_t s, const uint16_t *W, int n, int k, const uint16_t *x, int m,
                     void *y, int ldy, bool y_bf16, bool accumulate);
// the MFMA kernel alone (n a multiple of 128, k of 128, ldy of 4, 16-byte
// aligned operands, operands under 2 GiB: gemm_mfma_fits).  A plan names the
// workgroup tile (kTiles in gemm_mfma.hip: 0 128 x 128, 1 256 x 128, 2
// 128 x 256, 3 192 x 128, 4 192 x 256, 5 128 x 64, 6 128 x 96, features x
// tokens) and whether k is split in two;
// a split call needs a GemmSplitWs with room for gemm_split_bytes of partials
// and gemm_split_tiles tickets (zeroed once: every call leaves them zero),
// else it runs unsplit.
constexpr int kGemmTiles = 7;
struct GemmPlan {
    int tile;
    int split;  // 1 or 2
};
struct GemmSplitWs {
    void *part;
    size_t part_bytes;
    unsigned *ticket;  // tickets words of 32 unsigned each
    int tickets;
};
bool gemm_mfma_fits(const uint16_t *W, int n, int k, const uint16_t *x, int m, const void *y, int ldy);
int gemm_tile_by_name(const char *name);
GemmPlan gemm_mfma_plan(int n, int k, int m);
size_t gemm_split_bytes(int n, int m, GemmPlan p);
int gemm_split_tiles(int n, int m, GemmPlan p);
hipError_t gemm_bf16_mfma(const uint16_t *W, int n, int k, const uint16_t *x, int m, void *y, int ldy, bool y_bf16,
                          bool accumulate, hipStream_t s, GemmPlan p, const GemmSplitWs *ws);
// act[m][f] (rows ld elements apart) = silu(g) u, bf16, with g and u the
// bf16-rounded products x . Wg^T and x . Wu^T (Wg, Wu: [f][k]): the gate/up
// GEMM and rows_swiglu_bf16 in one launch of the MFMA kernel, unsplit (plan:
// the tile of the [gate; up] product, n = 2 f), the same bits as
// gemm_bf16_mfma's unsplit bf16 output followed by launch_rows_swiglu_bf16's
// 16-byte kernel.  f a multiple of 64; k, alignment and sizes as
// gemm_mfma_fits; ld a multiple of 8.
bool gemm_swiglu_fits(const uint16_t *Wg, const uint16_t *Wu, int f, int k, const uint16_t *x, int m,
                      const uint16_t *act, int ld);
hipError_t gemm_swiglu_mfma(const uint16_t *Wg, const uint16_t *Wu, int f, int k, const uint16_t *x, int m,
                            uint16_t *act, int ld, hipStream_t s, GemmPlan p);
// The state's fused gate/up + SwiGLU: runs it and returns true when the
// state's choice for the unfused calls -- the gate/up GEMM(s) into gu (bf16
// [m][2 f], as one [gate; up] matrix, or, separate, two [f][k] matrices) and
// launch_rows_swiglu_bf16 -- is the MFMA kernel unsplit for every GEMM and the
// 16-byte row kernel, so that the fused call's bits equal theirs; else returns
// false having enqueued nothing (the caller issues the unfused calls).
bool gemm_swiglu(GemmState *g, hipStream_t s, const uint16_t *Wg, const uint16_t *Wu, bool separate, int f, int k,
                 const uint16_t *x, int m, const uint16_t *gu, uint16_t *act, hipError_t &err);

}  // namespace hymt
