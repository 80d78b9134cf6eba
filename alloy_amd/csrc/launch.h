// Host-side launchers shared between the kernel translation units and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qformats.h"

namespace alloy {

enum Fmt : int { F_Q8_0 = 0, F_Q5_0 = 1, F_Q4_K = 2, F_Q6_K = 3, F_MLX = 4, F_Q8_0S = 5, F_Q5_0S = 6 };
enum Path : int { P_AUTO = 0, P_GEMV = 1, P_GEMV_MFMA = 2, P_GEMM = 3 };

// Routed-expert column tile record (ints): expert, first expert-sorted position,
// route count (<= 16), 0, then the token index of each of the 16 route slots.
constexpr int kTileInts = 20;

// Launch-shape knobs (0 = automatic choice).
struct Opts {
  int lanes_per_row = 0;   // dot2 GEMV: threads cooperating on one row (multiple of 16, <= 256)
  int grid_cap = 0;        // dot2 GEMV: max workgroups (grid-stride beyond)
  int row_groups = 0;      // MFMA GEMV: 16-row groups per workgroup (1, 2)
  int depth = 0;           // dot2 GEMV: rows of weights in flight per thread (2, 3, 4)
  int variant = 0;         // dot2 GEMV: 0 automatic, 1 register ring, 2 LDS-staged tiles, 4 aligned-load LDS tiles
  int splits = 0;          // Q4_K GEMM with a forced tile (variant >= 4): K splits (needs the workspace)
};

// Several weight matrices (same format and K) against one x in a single launch:
// each workgroup serves one matrix (block ranges b0[i] .. b0[i+1]).
constexpr int kMaxBatch = 8;
template <int NB>
struct WaveBatchT {
  int n;
  int b0[NB + 1];
  QArgs a[NB];
  void* y[NB];
  int64_t ldy[NB];
  int N[NB];
};
using WaveBatch = WaveBatchT<kMaxBatch>;

// M = 1 GEMV over b.n matrices in one launch (wave-row kernel);
// hipErrorNotSupported when that kernel does not take the shape.
hipError_t launch_gemv_batched(int fmt, const WaveBatch& b, const void* x, bool x_f32, bool y_f32,
                               const Opts& o, hipStream_t st);

// Rows ids[0..n_ids) of an N-row matrix decoded to fp32 (ids outside [0, N): zeros).
hipError_t launch_embedding(int fmt, const QArgs& a, const void* ids, bool ids64, int64_t n_ids, int64_t N,
                            float* out, hipStream_t st);

hipError_t launch_dequant(int fmt, const QArgs& a, void* out, bool out_f16, int64_t row0,
                          int64_t nrows, hipStream_t st);
// M = 1 GEMV with the rows copied through LDS by aligned 16-byte loads (GGUF wire
// formats; fp16 activations).  hipErrorNotSupported when the shape does not fit.
hipError_t launch_gemv_tile(int fmt, const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32, int64_t M,
                            int64_t N, const Opts& o, hipStream_t st);
hipError_t launch_gemv_dot2(int fmt, const QArgs& a, const void* x, bool x_f32, void* y,
                            bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st);
// 2 <= M <= 16.  ws (ws_bytes): optional fp32 workspace for a K-split plan,
// gemv_workspace_bytes() of it (0: no split); without it the plan has no split.
hipError_t launch_gemv_mfma(int fmt, const QArgs& a, const void* x, bool x_f32, void* y,
                            bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st,
                            void* ws = nullptr, int64_t ws_bytes = 0);
int64_t gemv_workspace_bytes(int fmt, int64_t M, int64_t N, int64_t K);
// y (M x N, mn = M N, a multiple of 4) = the sum of the S fp32 slices ws[s][mn] in
// slice order; ws 16-byte and y 16- (fp32) or 8-byte (fp16) aligned, else
// hipErrorNotSupported.
hipError_t launch_splitk_sum(const float* ws, int S, int64_t mn, void* y, bool y_f32, hipStream_t st);
// Prefill GEMM.  ws (ws_bytes): optional fp32 workspace for the Q4_K split-K plan,
// gemm_workspace_bytes() of it (0: no split); without it the plan has no split.
hipError_t launch_gemm(int fmt, const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32,
                       int64_t M, int64_t N, const Opts& o, void* ws, int64_t ws_bytes, hipStream_t st);
int64_t gemm_workspace_bytes(int fmt, int64_t M, int64_t N, int64_t K);

// Gated pair y = act(x G^T) * (x U^T) (act 0 silu, 1 gelu in tanh form): one fused
// launch when glu_fused_supported() (Q4_K / MLX, M <= 16, the shapes where it is
// faster), else two products into fp32 buffers and launch_glu_combine over them.
bool glu_fused_supported(int fmt, int64_t M, int64_t N, int64_t K, bool x_f32, int gs);
hipError_t launch_glu_fused(int fmt, int act, const QArgs& g, const QArgs& u, const void* x, bool x_f32,
                            void* y, bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st);
hipError_t launch_glu_combine(int act, const float* g, const float* u, void* y, bool y_f32, int64_t n,
                              hipStream_t st);

// Compute units of the current device, and the workgroups of `kern` (`threads` per
// workgroup, `lds` bytes of dynamic LDS) resident per compute unit on it: both
// queried once per (device, kernel, launch shape) and kept for the process.
int cu_count();
int resident_per_cu(const void* kern, int threads, size_t lds);

// The v_dot2 GEMV gives each thread at most 2 decode units of a 256-thread row:
// K <= 512 units per row.
inline int64_t max_k_dot2(int fmt) { return fmt == F_Q6_K ? 512 * 64 : 512 * 32; }

}  // namespace alloy
