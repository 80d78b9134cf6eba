// GEMV for M <= 8 activation rows over GGUF formats with unaligned blocks (Q6_K 210 B,
// Q5_0 22 B, Q8_0 34 B per block): the weight rows are copied through LDS so that
// global memory is read with aligned 16-byte loads only (once, whatever M), fp16
// activations.
//
// A lane-per-unit GEMV that reads such blocks straight from global memory needs a
// dozen 2- and 4-byte loads per unit (block starts are only 2-byte aligned), which
// caps it far below HBM bandwidth.  Here a tile of R = 4 consecutive rows (one per
// wave) is contiguous in memory and 16-byte aligned (checked on the host), so the
// workgroup loads it with 16-byte loads into registers, one tile ahead of the one
// being computed, and stores it to LDS; each wave then decodes its row from LDS
// (2-byte-aligned LDS reads are cheap) with its 64 lanes splitting the row's units.
// The activations are packed once per workgroup into per-(token, unit) records in
// LDS (the format's v_dot2 pair order plus 16-element sums), read back per unit, row
// and token.
// The grid is persistent (resident workgroups); workgroup bx walks tiles bx, bx +
// grid, ...; rows past N read as zeros (buffer loads past the end) and are not stored.

#include "gemv.h"
#include "launch.h"
#include "xs.h"

namespace alloy {

namespace {

constexpr int kTileRows = 4;    // one row per wave
constexpr int kMaxCpl = 12;     // 16-byte chunks per lane per tile (48 KiB tiles)
constexpr int kMaxTokens = 8;   // activation rows (records of each live in LDS)

template <class F>
constexpr int rec_words() {     // packed x record of one unit, in dwords (16-byte multiple)
  return ((F::UE / 2 + F::UE / 16) + 3) / 4 * 4;
}

}  // namespace

// (the arguments are scalars, which the dispatch preloads into SGPRs)
template <class F, typename YT>
__global__ __launch_bounds__(256) void k_gemv_t(const uint8_t* w, int64_t rbytes, int Kx, const f16* x, int M, YT* y,
                                                int N, int cpl, int ntiles) {
  extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
  const QArgs a{w, nullptr, nullptr, nullptr, rbytes, 0, Kx};
  constexpr int RW = rec_words<F>();
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
  const int K = a.K, U = K / F::UE;
  const uint32_t rb = (uint32_t)a.rb, tb = kTileRows * rb;
  uint32_t* xrec = (uint32_t*)sm;                                   // M x U records of RW dwords
  uint8_t* tile = sm + (uint32_t)(M * U) * RW * 4u;                 // cpl * 4 KiB
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)((uint32_t)N * rb), ALLOY_RSRC_DW3);
  const int grid = (int)gridDim.x;
  int tl = (int)blockIdx.x;

  // first tile's loads, then the activation records (their global reads overlap)
  u32x4 v[kMaxCpl];
  auto load_tile = [&](int tt) {
    const uint32_t base = tt < ntiles ? (uint32_t)tt * tb : 0x80000000u;
#pragma unroll
    for (int c = 0; c < kMaxCpl; ++c)
      if (c < cpl) {
        const uint32_t o = (uint32_t)c * 4096u + (uint32_t)t * 16u;
        v[c] = __builtin_amdgcn_raw_buffer_load_b128(wr, o < tb ? base + o : 0x80000000u, 0, kStream);
      }
  };
  load_tile(tl);
  for (int i = t; i < M * U; i += 256) {
    const int m = i / U, u = i - m * U;
    uint32_t xp[F::UE / 2];
    float xg[F::UE / 16];
    load_x_unit<F, f16>(x + (size_t)m * K, u, xp, xg);
    uint32_t* r = xrec + i * RW;
#pragma unroll
    for (int i = 0; i < F::UE / 2; i += 4) *(u32x4*)(r + i) = u32x4{xp[i], xp[i + 1], xp[i + 2], xp[i + 3]};
    float g4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < F::UE / 16; ++i) g4[i & 3] = xg[i];
    if constexpr (F::UE / 16 <= 4) {
      *(u32x4*)(r + F::UE / 2) = u32x4{__builtin_bit_cast(uint32_t, g4[0]), __builtin_bit_cast(uint32_t, g4[1]),
                                       __builtin_bit_cast(uint32_t, g4[2]), __builtin_bit_cast(uint32_t, g4[3])};
    }
  }

  constexpr uint32_t esz = sizeof(YT);
  const __amdgpu_buffer_rsrc_t yr =
      __builtin_amdgcn_make_buffer_rsrc((void*)y, (short)0, (int)((uint32_t)(M * N) * esz), ALLOY_RSRC_DW3);
  for (; tl < ntiles; tl += grid) {
#pragma unroll
    for (int c = 0; c < kMaxCpl; ++c)
      if (c < cpl) {
        const uint32_t o = (uint32_t)c * 4096u + (uint32_t)t * 16u;
        if (o < tb) *(u32x4*)(tile + o) = v[c];
      }
    load_tile(tl + grid);                 // next tile in flight during this one
    lds_barrier_asm();
    const uint8_t* row = tile + (uint32_t)wv * rb;
    const uint32_t n = (uint32_t)tl * kTileRows + (uint32_t)wv;
    // token by token: the row's units are decoded again per token from LDS (the
    // tile is read once from HBM whatever M is)
    for (int m = 0; m < M; ++m) {
      float acc = 0.f;
      for (int u = lane; u < U; u += 64) {
        const uint32_t* r = xrec + (m * U + u) * RW;
        uint32_t xp[F::UE / 2];
        float xg[F::UE / 16];
#pragma unroll
        for (int i = 0; i < F::UE / 2; i += 4) {
          const u32x4 q = *(const u32x4*)(r + i);
          xp[i] = q.x; xp[i + 1] = q.y; xp[i + 2] = q.z; xp[i + 3] = q.w;
        }
        const u32x4 g = *(const u32x4*)(r + F::UE / 2);
        // elements copied to scalars first: a bit_cast applied to a vector element
        // directly picks element 0 in this compiler
        const uint32_t g0 = g.x, g1 = g.y, g2 = g.z, g3 = g.w;
        const float gg[4] = {__builtin_bit_cast(float, g0), __builtin_bit_cast(float, g1),
                             __builtin_bit_cast(float, g2), __builtin_bit_cast(float, g3)};
#pragma unroll
        for (int i = 0; i < F::UE / 16; ++i) xg[i] = gg[i];
        acc += F::dot(F::load_row(row, u), u, xp, xg);
      }
      acc = dpp_sum_rows(acc, 6);
      const uint32_t yo = lane == 63 && n < (uint32_t)N ? ((uint32_t)m * (uint32_t)N + n) * esz : 0x80000000u;
      if constexpr (sizeof(YT) == 4) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), yr, yo, 0, 0);
      else __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16)acc), yr, yo, 0, 0);
    }
    lds_barrier_asm();                    // every wave is done with the tile in LDS
  }
}

// M = 1 over long rows: R = 1, 2 or 4 rows per tile so that the tile's units cover
// at least 192 of the 256 threads (thread t takes row t / (256 / R) and every
// (256 / R)-th unit of it), D tiles in flight in registers (ring slot = tile mod D),
// two LDS tile buffers and one barrier per tile.  Tiles stay within 16 KiB where
// k_gemv_t's four rows would pass its 48 KiB (Q8_0 rows of 14336 elements and
// longer).  Each wave's sum goes to LDS; the tile's rows are completed and stored
// after the next tile's barrier (the thread of row r sums its row's waves).
template <class F, typename YT, int D, int CPL>
__global__ __launch_bounds__(256) void k_gemv_rt(const uint8_t* w, int64_t rbytes, int Kx, const f16* x, YT* y,
                                                 int N, int R, int ntiles) {
  extern __shared__ __attribute__((aligned(16))) uint8_t sm[];
  constexpr int RW = rec_words<F>();
  constexpr uint32_t SLOT = (uint32_t)CPL * 4096u;
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
  const int K = Kx, U = K / F::UE;
  const uint32_t rb = (uint32_t)rbytes, tb = (uint32_t)R * rb;
  const int tpr = 256 / R, rt = t / tpr, j0 = t - rt * tpr, wpr = tpr >> 6;
  uint32_t* xrec = (uint32_t*)sm;                                   // U records of RW dwords
  uint8_t* tiles = sm + (uint32_t)U * RW * 4u;                      // two tile buffers
  float* part = (float*)(tiles + 2u * SLOT);                        // [2][4] wave sums
  const __amdgpu_buffer_rsrc_t wr =
      __builtin_amdgcn_make_buffer_rsrc((void*)w, (short)0, (int)((uint32_t)N * rb), ALLOY_RSRC_DW3);
  const int grid = (int)gridDim.x, bx = (int)blockIdx.x;
  const int nt = (ntiles - bx + grid - 1) / grid;                   // tiles of this workgroup (>= 1)

  u32x4 v[D][CPL];
  auto issue = [&](auto S, int i) {                                 // tile i of this workgroup -> ring slot S
    constexpr int s = decltype(S)::value;
    const uint32_t base = i < nt ? (uint32_t)(bx + i * grid) * tb : 0x80000000u;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t o = (uint32_t)c * 4096u + (uint32_t)t * 16u;
      v[s][c] = __builtin_amdgcn_raw_buffer_load_b128(wr, o < tb ? base + o : 0x80000000u, 0, kStream);
    }
  };
  auto finish = [&](int i) {                                        // rows of tile i from the wave sums
    if (t < R) {
      const float* p = part + 4 * (i & 1) + t * wpr;
      float sum = p[0];
      for (int k = 1; k < wpr; ++k) sum += p[k];
      const int n = (bx + i * grid) * R + t;
      if (n < N) y[n] = (YT)sum;
    }
  };
  auto step = [&](auto S, int i) {
    constexpr int s = decltype(S)::value;
    uint8_t* buf = tiles + (uint32_t)(i & 1) * SLOT;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const uint32_t o = (uint32_t)c * 4096u + (uint32_t)t * 16u;
      if (o < tb) *(u32x4*)(buf + o) = v[s][c];
    }
    issue(S, i + D);                                                // D tiles ahead, same slot
    lds_barrier_asm();                  // tile i in LDS; tile i - 1 decoded, its wave sums in LDS
    if (i > 0) finish(i - 1);
    const uint8_t* row = buf + (uint32_t)rt * rb;
    float acc = 0.f;
    for (int u = j0; u < U; u += tpr) {
      const uint32_t* r = xrec + u * RW;
      uint32_t xp[F::UE / 2];
      float xg[F::UE / 16];
#pragma unroll
      for (int k = 0; k < F::UE / 2; k += 4) {
        const u32x4 q = *(const u32x4*)(r + k);
        xp[k] = q.x; xp[k + 1] = q.y; xp[k + 2] = q.z; xp[k + 3] = q.w;
      }
      const u32x4 g = *(const u32x4*)(r + F::UE / 2);
      const uint32_t g0 = g.x, g1 = g.y, g2 = g.z, g3 = g.w;
      const float gg[4] = {__builtin_bit_cast(float, g0), __builtin_bit_cast(float, g1),
                           __builtin_bit_cast(float, g2), __builtin_bit_cast(float, g3)};
#pragma unroll
      for (int k = 0; k < F::UE / 16; ++k) xg[k] = gg[k];
      acc += F::dot(F::load_row(row, u), u, xp, xg);
    }
    acc = dpp_sum_rows(acc, 6);
    if (lane == 63) part[4 * (i & 1) + wv] = acc;
  };

  // the first D tiles' loads, then the activation records (their global reads overlap)
  issue(std::integral_constant<int, 0>{}, 0);
  if constexpr (D > 1) issue(std::integral_constant<int, 1>{}, 1);
  if constexpr (D > 2) issue(std::integral_constant<int, 2>{}, 2);
  if constexpr (D > 3) issue(std::integral_constant<int, 3>{}, 3);
  for (int i = t; i < U; i += 256) {
    uint32_t xp[F::UE / 2];
    float xg[F::UE / 16];
    load_x_unit<F, f16>(x, i, xp, xg);
    uint32_t* r = xrec + i * RW;
#pragma unroll
    for (int k = 0; k < F::UE / 2; k += 4) *(u32x4*)(r + k) = u32x4{xp[k], xp[k + 1], xp[k + 2], xp[k + 3]};
    float g4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < F::UE / 16; ++k) g4[k & 3] = xg[k];
    *(u32x4*)(r + F::UE / 2) = u32x4{__builtin_bit_cast(uint32_t, g4[0]), __builtin_bit_cast(uint32_t, g4[1]),
                                     __builtin_bit_cast(uint32_t, g4[2]), __builtin_bit_cast(uint32_t, g4[3])};
  }
  lds_barrier_asm();                                                // records complete

  static_assert(D >= 1 && D <= 4, "ring depth");
  for (int i = 0; i < nt; i += D) {     // unrolled by D: every ring slot index is a constant
    step(std::integral_constant<int, 0>{}, i);
    if constexpr (D > 1) { if (i + 1 >= nt) break; step(std::integral_constant<int, 1>{}, i + 1); }
    if constexpr (D > 2) { if (i + 2 >= nt) break; step(std::integral_constant<int, 2>{}, i + 2); }
    if constexpr (D > 3) { if (i + 3 >= nt) break; step(std::integral_constant<int, 3>{}, i + 3); }
  }
  lds_barrier_asm();                                                // the last tile's wave sums
  finish(nt - 1);
}

namespace {

template <class F>
hipError_t run_tile(const QArgs& a, const void* x, void* y, bool y_f32, int64_t M, int64_t N64, const Opts& o,
                    hipStream_t st) {
  static_assert(F::UE / 16 <= 4, "packed x record holds at most four sums");
  const int64_t tb = (int64_t)kTileRows * a.rb;
  if (a.K % 256 || tb % 16 || ((uintptr_t)a.w & 15) || ((uintptr_t)x & 15)) return hipErrorNotSupported;
  if ((uint64_t)N64 * (uint64_t)a.rb >= (1ull << 31) - (1u << 20)) return hipErrorNotSupported;
  const int cpl = (int)((tb + 4095) / 4096);
  const int U = a.K / F::UE;
  if ((uint64_t)M * (uint64_t)N64 * 4u >= (1ull << 31)) return hipErrorNotSupported;
  const size_t lds = (size_t)M * U * rec_words<F>() * 4 + (size_t)cpl * 4096;
  if (cpl > kMaxCpl || lds > 160 * 1024) return hipErrorNotSupported;
  const int N = (int)N64;
  const int ntiles = (N + kTileRows - 1) / kTileRows;
  const void* k = y_f32 ? (const void*)k_gemv_t<F, float> : (const void*)k_gemv_t<F, f16>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  int grid = resident_per_cu(k, 256, lds) * cu_count();
  if (o.grid_cap > 0 && o.grid_cap < grid) grid = o.grid_cap;
  if (grid > ntiles) grid = ntiles;
  if (y_f32)
    hipLaunchKernelGGL((k_gemv_t<F, float>), dim3((unsigned)grid), dim3(256), lds, st, a.w, a.rb, a.K, (const f16*)x, (int)M,
                       (float*)y, N, cpl, ntiles);
  else
    hipLaunchKernelGGL((k_gemv_t<F, f16>), dim3((unsigned)grid), dim3(256), lds, st, a.w, a.rb, a.K, (const f16*)x, (int)M,
                       (f16*)y, N, cpl, ntiles);
  return hipGetLastError();
}

template <class F, typename YT, int D>
hipError_t launch_rt(int cpl, const QArgs& a, const void* x, void* y, int N, int R, int ntiles, size_t lds, int cap,
                     hipStream_t st) {
  const void* k = cpl == 1 ? (const void*)k_gemv_rt<F, YT, D, 1> : cpl == 2 ? (const void*)k_gemv_rt<F, YT, D, 2>
                : cpl == 3 ? (const void*)k_gemv_rt<F, YT, D, 3> : (const void*)k_gemv_rt<F, YT, D, 4>;
  if (lds > 65536) {
    const hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  int grid = resident_per_cu(k, 256, lds) * cu_count();
  if (cap > 0 && cap < grid) grid = cap;
  if (grid > ntiles) grid = ntiles;
  if (grid < 1) return hipErrorNotSupported;
  void* args[] = {(void*)&a.w, (void*)&a.rb, (void*)&a.K, (void*)&x, (void*)&y, (void*)&N, (void*)&R, (void*)&ntiles};
  return hipLaunchKernel(k, dim3((unsigned)grid), dim3(256), args, lds, st);
}

// M = 1 through k_gemv_rt; hipErrorNotSupported for rows of fewer than 64 units or
// tiles over 16 KiB.
template <class F>
hipError_t run_ring(const QArgs& a, const void* x, void* y, bool y_f32, int64_t N64, const Opts& o, hipStream_t st) {
  const int U = a.K / F::UE;
  if (a.K % 256 || U < 64 || ((uintptr_t)a.w & 15) || ((uintptr_t)x & 15)) return hipErrorNotSupported;
  const int R = U >= 192 ? 1 : U >= 96 ? 2 : 4;                      // at least 3/4 of the threads busy
  const int64_t tb = (int64_t)R * a.rb;
  if (tb % 16 || tb > 4 * 4096) return hipErrorNotSupported;
  if ((uint64_t)N64 * (uint64_t)a.rb >= (1ull << 31) - (1u << 20)) return hipErrorNotSupported;
  const int cpl = (int)((tb + 4095) / 4096);
  const size_t lds = (size_t)U * rec_words<F>() * 4 + (size_t)cpl * 2 * 4096 + 32;
  if (lds > 160 * 1024) return hipErrorNotSupported;
  const int N = (int)N64, ntiles = (N + R - 1) / R;
  const int D = o.depth >= 4 ? 4 : 2;                               // two tiles in flight by default
  if (y_f32)
    return D == 2 ? launch_rt<F, float, 2>(cpl, a, x, y, N, R, ntiles, lds, o.grid_cap, st)
                  : launch_rt<F, float, 4>(cpl, a, x, y, N, R, ntiles, lds, o.grid_cap, st);
  return D == 2 ? launch_rt<F, f16, 2>(cpl, a, x, y, N, R, ntiles, lds, o.grid_cap, st)
                : launch_rt<F, f16, 4>(cpl, a, x, y, N, R, ntiles, lds, o.grid_cap, st);
}

}  // namespace

hipError_t launch_gemv_tile(int fmt, const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32, int64_t M,
                            int64_t N, const Opts& o, hipStream_t st) {
  if (M < 1 || M > kMaxTokens || x_f32) return hipErrorNotSupported;
  if (N == 0) return hipSuccess;
  // M = 1: the tile ring on Q6_K rows of 12288 elements or more (one row per tile;
  // 14336 x 4096: 15.4 vs 16.0 us) and where the four-row tile would pass 48 KiB
  // (Q8_0 14336 x 4096: 15.3 us against 21.6 us on the wave-row fallback), else the
  // four-row tile kernel (equal or faster on the other BASELINE shapes, e.g. Q6_K
  // 4096 x 4096 6.1 vs 6.7 us); depth 2..4 forces the ring, 1 the four-row tile
  const bool ring_ok = M == 1 && o.depth != 1 && (fmt == F_Q6_K || fmt == F_Q5_0 || fmt == F_Q8_0);
  auto ring = [&]() {
    return fmt == F_Q6_K ? run_ring<FQ6K>(a, x, y, y_f32, N, o, st)
         : fmt == F_Q5_0 ? run_ring<FQ50>(a, x, y, y_f32, N, o, st)
                         : run_ring<FQ80>(a, x, y, y_f32, N, o, st);
  };
  if (ring_ok && (o.depth >= 2 || (fmt == F_Q6_K && a.K >= 12288))) {
    const hipError_t e = ring();
    if (e != hipErrorNotSupported) return e;
  }
  hipError_t e;
  switch (fmt) {
    case F_Q6_K: e = run_tile<FQ6K>(a, x, y, y_f32, M, N, o, st); break;
    case F_Q5_0: e = run_tile<FQ50>(a, x, y, y_f32, M, N, o, st); break;
    case F_Q8_0: e = run_tile<FQ80>(a, x, y, y_f32, M, N, o, st); break;
    case F_Q4_K: e = run_tile<FQ4K>(a, x, y, y_f32, M, N, o, st); break;
    default: return hipErrorNotSupported;
  }
  return e == hipErrorNotSupported && ring_ok ? ring() : e;
}

}  // namespace alloy
