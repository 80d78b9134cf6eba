// Routed-expert MoE over MLX 4-bit or GGUF (Q4_K gate/up, Q6_K down) experts:
// workspace layout and launchers.
#pragma once
#include "launch.h"

namespace alloy {

constexpr int kMoeMaxExperts = 1024;
constexpr int kMoeMaxTopK = 32;
constexpr int kMoeMaxRoutes = 1 << 20;   // T * top_k
constexpr int kMoeColTile = 16;          // routed rows per grouped-GEMV column tile

// Byte offsets into the caller's workspace (every region 256-byte aligned).
struct MoeLayout {
  int64_t R = 0;          // routes = T * top_k
  int64_t max_tiles = 0;  // upper bound on column tiles: min(E, R) + ceil(R / 16)
  size_t idx = 0;         // i32[R]   expert per route (route r = t*top_k + s)
  size_t wts = 0;         // f32[R]   routing weight per route
  size_t sorted = 0;      // i32[R]   expert-sorted position -> route (stable)
  size_t inv = 0;         // i32[R]   route -> expert-sorted position
  size_t tiles = 0;       // i32[max_tiles][4]: expert, first sorted position, count, pad
  size_t ntiles = 0;      // i32[1]   number of valid tiles
  size_t h = 0;           // f32[R][I]  silu(gate) * up per sorted position (xs path);
                          // f32[R][2I] gate | up per route (routed wave path)
  size_t part = 0;        // f32[R][H]  down projection per sorted position
  size_t total = 0;
};

MoeLayout moe_layout(int64_t T, int E, int top_k, int64_t H, int64_t I);

struct MoeArgs {
  const f16* x;          // [T, H]
  const float* logits;   // [T, E]
  QArgs gu;              // rows E*2I of K = H
  QArgs dn;              // rows E*H  of K = I
  int E, top_k;
  int64_t T, H, I;
  uint8_t* ws;
  float* y;              // [T, H]
};

hipError_t launch_router(const float* logits, int32_t* idx, float* w, int64_t T, int E, int top_k,
                         hipStream_t st);
hipError_t launch_mlx_moe(const MoeArgs& m, const MoeLayout& L, hipStream_t st);
// GGUF experts: gate/up Q4_K (gu.rb = H/256*144), down Q6_K (dn.rb = I/256*210).
bool gguf_moe_supported(int64_t T, int64_t H, int64_t I, const MoeLayout& L);
hipError_t launch_gguf_moe(const MoeArgs& m, const MoeLayout& L, hipStream_t st);

}  // namespace alloy
