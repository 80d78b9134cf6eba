// Helpers of the GEMV / GEMM kernels: activation loading into the formats' v_dot2
// pair order, the DPP row reductions, an LDS-only workgroup barrier, and the
// v_fma_mix dequant steps of the Q4_K GEMMs.
#pragma once
#include <type_traits>
#include <utility>

#include "qformats.h"

namespace alloy {

// Formats whose wave-path raw loads are completed across lanes before the dot
// (F::share), e.g. a header loaded a dword per lane.
template <class F, class = void>
struct HasShare : std::false_type {};
template <class F>
struct HasShare<F, std::void_t<decltype(F::share(std::declval<typename F::Raw&>()))>> : std::true_type {};
// Formats with a pair-split dot for the wave-row GEMV (F::dot_pair, F::pair_x_sums).
template <class F, class = void>
struct HasPairDot : std::false_type {};
template <class F>
struct HasPairDot<F, std::void_t<decltype(F::pair_x_sums((float*)nullptr, false))>> : std::true_type {};

// Workgroup barriers that order LDS only (lgkmcnt(0) before s_barrier, nothing
// else), so global loads still in flight (a GEMV's weight prefetch) are not drained
// at the barrier, as a __syncthreads fence would.
//
// lds_barrier: release / acquire fences restricted to the local address space.
// Builtins, so the compiler's hazard checks (the wait states between an MFMA and a
// read of its result) stay complete around it: the barrier of MFMA kernels.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
// lds_barrier_asm: the same as inline asm with a memory clobber, which also keeps the
// global loads issued before it in place (the fences above let the scheduler sink a
// weight prefetch below the barrier, measured 7-10 % slower on the M = 1 GEMV).  The
// asm hides the instructions from the hazard checks: only for kernels without MFMAs.
__device__ __forceinline__ void lds_barrier_asm() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// y[i] = v as fp32 or RN16
__device__ __forceinline__ void store_y(void* y, bool y_f32, int64_t i, float v) {
  if (y_f32) ((float*)y)[i] = v;
  else ((f16*)y)[i] = (f16)v;
}

// elements k0..k0+31 of row n as RN16 of their exact fp32 values
template <class F>
__device__ __forceinline__ void dec32_f16(const QArgs& a, int64_t n, int k0, f16x8 (&o)[4]) {
  float w[32];
  F::dec32(a, n, k0, w);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[j][e] = (f16)w[8 * j + e];   // RNE
}

template <typename XT>
__device__ __forceinline__ f16x8 ld_x8(const XT* p);
template <>
__device__ __forceinline__ f16x8 ld_x8<f16>(const f16* p) { return *(const f16x8*)p; }
template <>
__device__ __forceinline__ f16x8 ld_x8<float>(const float* p) {
  const f32x4 a = *(const f32x4*)p, b = *(const f32x4*)(p + 4);
  f16x8 r;
  r[0] = (f16)a[0]; r[1] = (f16)a[1]; r[2] = (f16)a[2]; r[3] = (f16)a[3];
  r[4] = (f16)b[0]; r[5] = (f16)b[1]; r[6] = (f16)b[2]; r[7] = (f16)b[3];
  return r;
}

__device__ __forceinline__ uint32_t pack2(f16 lo, f16 hi) {
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

template <class F, typename XT>
__device__ __forceinline__ void load_x_unit(const XT* x, int u, uint32_t (&xr)[F::UE / 2],
                                            float (&xg)[F::UE / 16]) {
  constexpr int RUN = F::RUN;
#pragma unroll
  for (int r = 0; r < F::UE / RUN; ++r) {
    const XT* p = x + F::run_start(u, r);
    f16 v[RUN];
#pragma unroll
    for (int c = 0; c < RUN / 8; ++c) {
      const f16x8 t = ld_x8<XT>(p + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * c + e] = t[e];
    }
    uint32_t* o = xr + (RUN / 2) * r;
    if (F::XPERM == 4) {
#pragma unroll
      for (int j = 0; j < RUN / 4; ++j) {
        o[2 * j] = pack2(v[4 * j], v[4 * j + 2]);
        o[2 * j + 1] = pack2(v[4 * j + 1], v[4 * j + 3]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < RUN / 8; ++j) {
        const int b = 8 * j;
        o[4 * j] = pack2(v[b], v[b + 4]);
        o[4 * j + 1] = pack2(v[b + 2], v[b + 6]);
        o[4 * j + 2] = pack2(v[b + 1], v[b + 5]);
        o[4 * j + 3] = pack2(v[b + 3], v[b + 7]);
      }
    }
    // per-16-element sums: pairs 8h..8h+7 hold exactly elements 16h..16h+15 in
    // either order; v_dot2 against (1, 1) adds them in fp32 without conversions
#pragma unroll
    for (int h = 0; h < RUN / 16; ++h) {
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 8; ++q) sum = dot2(o[8 * h + q], MAGIC1, sum);
      xg[(RUN / 16) * r + h] = sum;
    }
  }
}

// Row-sum reduction across the L = 16, 32 or 64 lanes that share a row inside one
// wave (DPP quad_perm, row mirrors, row_bcast 15/31) — no LDS, no barrier.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, ROW_MASK, 0xF, false));
}
// Sum over groups of 1 << lshift lanes (16, 32 or 64); the total is complete in the
// group's last lane.  Branch-free in lshift, so the loop body has no control flow.
__device__ __forceinline__ float dpp_sum_rows(float v, int lshift) {
  v += dpp_f<0xB1, 0xF>(v);     // quad_perm [1,0,3,2]
  v += dpp_f<0x4E, 0xF>(v);     // quad_perm [2,3,0,1]
  v += dpp_f<0x141, 0xF>(v);    // row_half_mirror: 8-lane sums
  v += dpp_f<0x140, 0xF>(v);    // row_mirror: every lane of a 16-lane row holds its sum
  const float s32 = v + dpp_f<0x142, 0xA>(v);        // row_bcast:15 -> rows 1, 3: 32-lane sums
  const float s64 = s32 + dpp_f<0x143, 0xC>(s32);    // row_bcast:31 -> row 3: 64-lane sum
  return lshift == 4 ? v : lshift == 5 ? s32 : s64;
}

}  // namespace alloy
