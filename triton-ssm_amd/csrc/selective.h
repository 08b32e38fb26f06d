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
  float* T = nullptr;  // [nbatch][nch][Dc] (or [nbatch][nch]) dt sums per chunk
};

// Steps per chunk for these sizes (0: the three-pass scan does not apply).
int64_t sel_chunk_steps(int64_t nbatch, int64_t L, int64_t Dc);

// Workspace bytes of the three-pass scan (0 if it does not apply to the shape).
int64_t sel_chunked_bytes(int64_t nbatch, int64_t L, int64_t Dc, int64_t N);

// Launch the three passes on `s`.  dtype F32 or BF16, N 8 or 16; dt shared by
// the channels (sdt_d unused) or per channel (then not timestamps).
int sel_chunked_launch(int dtype, int disc, bool dt_shared, bool tau, const SelPtrs& p,
                       int64_t nbatch, int64_t L, int64_t Dc, int64_t N, int64_t sx_b,
                       int64_t sx_l, int64_t sdt_b, int64_t sdt_l, int64_t sdt_d, int64_t sB_b,
                       int64_t sB_l, int64_t sC_b, int64_t sC_l, int64_t sy_b, int64_t sy_l,
                       hipStream_t s);

}  // namespace tssm
