// Host interface of the three-pass Mamba-1 selective scan (selective.hip),
// used by tssm_selective_scan for large problems with N = 8 or 16 states.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tssm {

// Steps per chunk of the three-pass scan.
constexpr int64_t kSelChunkSteps = 32;
// Smallest problem (waves of 64 channels x one chunk) given to it; smaller
// ones keep the single-pass kernel.
constexpr int64_t kSelMinWaves = 512;

struct SelPtrs {
  const void* x = nullptr;
  const float* dt = nullptr;
  const float* A_log = nullptr;
  const void* B = nullptr;
  const void* C = nullptr;
  const float* D = nullptr;
  const float* h0 = nullptr;
  void* y = nullptr;
  float* h_last = nullptr;
  float* S = nullptr;  // [nbatch][nch][Dc][N] chunk end states -> entry states
  float* T = nullptr;  // [nbatch][nch][Dc] (or [nbatch][nch]) dt sums per chunk,
                       // followed by the carry pass's segment block (sel_state_floats)
  // dt produced in the passes (W != NULL): `dt` then holds the raw rows
  // [nbatch][L][rank] (strides sdt_b, sdt_l, 1) and
  // dt[b,t,d] = clamp(softplus(sum_q raw[b,t,q] W[q,d] + bias[d]), dt_min, dt_max)
  const float* W = nullptr;     // [rank][Dc], row stride sw_r
  const float* bias = nullptr;  // [Dc]
  int64_t sw_r = 0;
  int64_t rank = 0;
  float dt_min = 0.0f, dt_max = 0.0f;
  // optional [nbatch][L][Dc] table: pass 1 stores the dt it produced there and
  // pass 3 reads it back (NULL: pass 3 produces dt again)
  float* dtw = nullptr;
};

// Whether the three-pass scan can produce dt itself for these operands: the
// matrix-core form needs 16-byte rows (rank, Dc, row strides multiples of 4;
// raw rows, W and bias 16-byte aligned) and rank <= kSelMaxRank.
constexpr int64_t kSelMaxRank = 64;
bool sel_proj_ok(const float* raw, const float* W, const float* bias, int64_t Dc, int64_t rank,
                 int64_t sr_b, int64_t sr_l, int64_t sw_r);

// Steps per chunk for these sizes (0: the three-pass scan does not apply).
int64_t sel_chunk_steps(int64_t nbatch, int64_t L, int64_t Dc);

// Chunks per segment when the carry pass splits a long sequence into segments
// (few (batch, channel, state) lanes, many chunks).
constexpr int64_t kSelSegChunks = 32;

// Floats of the chunk-state block at SelPtrs::S: chunk end states
// [nbatch][nch][Dc][N], dt sums [nbatch][nch][Dc], then the segment states
// [nbatch][nseg][Dc][N] and segment dt sums [nbatch][nseg][Dc],
// nseg = ceil(nch / kSelSegChunks).
int64_t sel_state_floats(int64_t nbatch, int64_t nch, int64_t Dc, int64_t N);

// Workspace bytes of the three-pass scan (0 if it does not apply to the shape).
int64_t sel_chunked_bytes(int64_t nbatch, int64_t L, int64_t Dc, int64_t N);

// Bytes of the produced-dt table (SelPtrs::dtw).
int64_t sel_dt_table_bytes(int64_t nbatch, int64_t L, int64_t Dc);

// Launch the three passes on `s`.  dtype F32 or BF16, N 8 or 16; dt shared by
// the channels (sdt_d unused), per channel (then not timestamps), or produced
// from raw rows (p.W set; sel_proj_ok must hold; dt_shared and tau false).
int sel_chunked_launch(int dtype, int disc, bool dt_shared, bool tau, const SelPtrs& p,
                       int64_t nbatch, int64_t L, int64_t Dc, int64_t N, int64_t sx_b,
                       int64_t sx_l, int64_t sdt_b, int64_t sdt_l, int64_t sdt_d, int64_t sB_b,
                       int64_t sB_l, int64_t sC_b, int64_t sC_l, int64_t sy_b, int64_t sy_l,
                       hipStream_t s);

// Whether the interpolation can be formed inside pass 1 (sel_interp_launch):
// fp32/bf16 I/O, N 8 or 16, fp32 masks in 16-byte rows, FTILE a power of two
// in [16, 256], 1 <= K <= 64, F a multiple of 4, a problem the three passes
// take, V's row stride small enough for 32-bit row offsets within a chunk.
bool sel_interp_ok(int dtype, int64_t nbatch, int64_t T, int64_t F, int64_t N, int64_t K,
                   int64_t FTILE, const void* M, int64_t sm_b, int64_t sm_t, int64_t sv_t);

}  // namespace tssm
