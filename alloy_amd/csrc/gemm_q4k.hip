// Q4_K prefill GEMM, one wave per SIMD: y[M,N] = x[M,K] (fp16) . dequant(W)[N,K]^T.
//
// 256 threads = 4 waves as 2 (x rows) x 2 (weight rows); each wave owns a
// 32MI x 32NI output block (4 x 4 tiles of v_mfma_f32_32x32x16_f16 at 256 x 256, 256
// fp32 accumulators, which live in the accumulator half of the register file at one
// wave per SIMD).  Against the 8-wave kernel this halves the LDS operand reads per
// MFMA (a 128 x 128 wave block reads 8 fragments per 16 MFMAs instead of 6 per 8).
// K advances in steps of 64 through double-buffered LDS (x tile and dequantised weight
// tile, rows padded to 72 halves; 144 KB at 256 x 256) with one barrier per step:
// step kt multiplies from buffer kt%2 while the weights of step kt+1 are dequantised
// into the other buffer in quarters between its MFMA groups, and the x chunks of step
// kt+1 (loaded at the start of the step) are stored after slice 1.  Buffer-resource loads read
// rows past M or N as zero and stores past them are dropped.
//
// Weight dequant: the nibbles are masked into the halves of a dword as fp16
// denormals q*2^-24 (16q*2^-24 for high nibbles); v_fma_mix_f32 forms
// d*sc*q - dmin*m with the scale pre-multiplied by 2^24 (2^20), which is the exact
// product rounded once to fp32 — the fp32 weight — and v_cvt_pk_f16_f32 rounds it to
// fp16.  Plain C: the compiler selects both instructions and sees every register they
// write, so its MFMA hazard checks stay complete.
#include <type_traits>

#include "gemv.h"
#include "launch.h"

namespace alloy {

namespace {

constexpr int WBK = 64, WLD = 72;

__device__ __forceinline__ f16 mixh(uint32_t q, int hi, float s, float c) {
  const f16 h = __builtin_bit_cast(f16, (uint16_t)(hi ? (q >> 16) : (q & 0xFFFFu)));
  return (f16)__builtin_fmaf((float)h, s, c);
}

// 8 weights of one dword of quant bytes: its low nibbles (scale s0/c0) and high
// nibbles (s1/c1), each as 4 fp16 in byte order.
__device__ __forceinline__ void deq_dword(uint32_t w, const float (&s)[2], const float (&c)[2], uint2& lo,
                                          uint2& hi) {
  const uint32_t w8 = w >> 8;
  const uint32_t la = w & 0x000F000Fu, lb = w8 & 0x000F000Fu;   // bytes (0, 2), (1, 3)
  const uint32_t ha = w & 0x00F000F0u, hb = w8 & 0x00F000F0u;
  const f16x2 l0 = {mixh(la, 0, s[0], c[0]), mixh(lb, 0, s[0], c[0])};
  const f16x2 l1 = {mixh(la, 1, s[0], c[0]), mixh(lb, 1, s[0], c[0])};
  const f16x2 h0 = {mixh(ha, 0, s[1], c[1]), mixh(hb, 0, s[1], c[1])};
  const f16x2 h1 = {mixh(ha, 1, s[1], c[1]), mixh(hb, 1, s[1], c[1])};
  lo = uint2{__builtin_bit_cast(uint32_t, l0), __builtin_bit_cast(uint32_t, l1)};
  hi = uint2{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
}

}  // namespace

// MI x NI: 32x32 MFMA tiles per wave; workgroup tile QBM = 64*MI x QBN = 64*NI.
// TPR = 256/QBN threads share a weight row (1 at QBN = 256, 2 at QBN = 128).
// nsb > 0: split K — blockIdx.z covers super-blocks [z*nsb, (z+1)*nsb) and writes its
// fp32 partial tile to slice z of y.  remap: workgroups are spread over the 8 XCDs
// round-robin; remap != 0 gives each XCD a contiguous range of (m, n) tiles so the
// x rows it reads stay in its L2.
template <int MI, int NI, typename YT>
__global__ __launch_bounds__(256) void k_gemm_q4k_w4(QArgs a, const f16* x, int M, YT* y, int N, int nsb,
                                                     int remap) {
  constexpr int QBM = 64 * MI, QBN = 64 * NI, AC = QBM / 32, TPR = 256 / QBN, QC = 2 / TPR;
  static_assert(TPR == 1 || TPR == 2, "weight tile must be 128 or 256 rows");
  __shared__ __attribute__((aligned(16))) f16 As[2][QBM][WLD];
  __shared__ __attribute__((aligned(16))) f16 Bs[2][QBN][WLD];
  const int K = a.K, KT = nsb > 0 ? 4 * nsb : K / WBK;
  const uint32_t kb = nsb > 0 ? (uint32_t)blockIdx.z * (uint32_t)nsb : 0u;
  if (nsb > 0) y += (size_t)blockIdx.z * (size_t)M * (size_t)N;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  int bx = (int)blockIdx.x, by = (int)blockIdx.y;
  if (remap) {
    const int gx = (int)gridDim.x, tiles = gx * (int)gridDim.y, bid = by * gx + bx;
    const int t = (bid & 7) * (tiles >> 3) + (bid >> 3);   // tiles % 8 == 0 (host)
    bx = t % gx;
    by = t / gx;
  }
  const int m0 = by * QBM, n0 = bx * QBN;
  const uint32_t rb = (uint32_t)a.rb;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), ALLOY_RSRC_DW3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.w, (short)0, (int)((uint32_t)N * rb), ALLOY_RSRC_DW3);
  // x tile: QBM rows x 8 chunks of 16 B, AC chunks per thread (8 threads per row)
  uint32_t xoff[AC];
  int arow[AC], acol[AC];
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int c = tid + 256 * i;
    arow[i] = c >> 3;
    acol[i] = (c & 7) * 8;
    xoff[i] = ((uint32_t)(m0 + arow[i]) * (uint32_t)K + 256u * kb + (uint32_t)acol[i]) * 2u;
  }
  // weight tile: thread owns row br and quant chunks bh*QC .. bh*QC+QC-1 (16 B each) of
  // every 32-byte pair: chunk k holds elements 16k + [0,16) (low nibbles, sub-block
  // 2p) and 32 + 16k + [0,16) (high nibbles, sub-block 2p+1) of the pair's step.
  const int br = tid / TPR, bh = tid % TPR;
  const uint32_t wrow = (uint32_t)(n0 + br) * rb + 144u * kb;

  struct Blk { u32x4 hd, q[4 * QC]; };     // this thread's bytes of one super-block
  auto bload = [&](int sb, Blk& r) {       // past the end: in-bounds garbage or zeros
    const uint32_t so = (uint32_t)sb * 144u;
    r.hd = __builtin_amdgcn_raw_buffer_load_b128(wr, wrow, so, 0);
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int k = 0; k < QC; ++k)
        r.q[QC * p + k] =
            __builtin_amdgcn_raw_buffer_load_b128(wr, wrow + 16u + 32u * p + 16u * (uint32_t)(QC * bh + k), so, 0);
  };
  u32x4 xs[AC];
  auto xload = [&](int kt) {               // the step offset is uniform: scalar operand
    const uint32_t so = 2u * (uint32_t)kt * WBK;
#pragma unroll
    for (int i = 0; i < AC; ++i) xs[i] = __builtin_amdgcn_raw_buffer_load_b128(xr, xoff[i], so, 0);
  };
  auto scales = [&](const Blk& r, int p, float (&s)[2], float (&c)[2]) {
    uint32_t sc0, mn0, sc1, mn1;
    q4k_scale_min(r.hd.y, r.hd.z, r.hd.w, 2 * p, sc0, mn0);     // p is a constant
    q4k_scale_min(r.hd.y, r.hd.z, r.hd.w, 2 * p + 1, sc1, mn1);
    const float d = h2f(r.hd.x), dmin = h2f(r.hd.x >> 16);
    s[0] = d * (float)sc0 * 16777216.f;                 // 2^24
    s[1] = d * (float)sc1 * 1048576.f;                  // 2^24 / 16
    c[0] = -(dmin * (float)mn0);
    c[1] = -(dmin * (float)mn1);
  };
  // quarter j of a step's dequant: QC dwords -> 4*QC elements of each sub-block
  auto deq = [&](const Blk& r, int p, int j, const float (&s)[2], const float (&c)[2], int buf) {
    if constexpr (QC == 2) {               // dwords 2j, 2j+1 of the pair: bytes 8j .. 8j+7
      const u32x4& q = r.q[2 * p + (j >> 1)];
      const uint32_t w0 = (j & 1) ? q.z : q.x, w1 = (j & 1) ? q.w : q.y;
      uint2 l0, h0, l1, h1;
      deq_dword(w0, s, c, l0, h0);
      deq_dword(w1, s, c, l1, h1);
      *(u32x4*)&Bs[buf][br][8 * j] = u32x4{l0.x, l0.y, l1.x, l1.y};
      *(u32x4*)&Bs[buf][br][32 + 8 * j] = u32x4{h0.x, h0.y, h1.x, h1.y};
    } else {                               // dword j of chunk bh: bytes 16bh + 4j .. +3
      const u32x4& q = r.q[p];
      const uint32_t w = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
      uint2 l, h;
      deq_dword(w, s, c, l, h);
      *(uint2*)&Bs[buf][br][16 * bh + 4 * j] = l;
      *(uint2*)&Bs[buf][br][32 + 16 * bh + 4 * j] = h;
    }
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // A/B fragments of K slice ks of buffer buf for this wave's tiles
  auto frags = [&](int buf, int ks, f16x8 (&af)[MI], f16x8 (&bf)[NI]) {
    const int kc = 16 * ks + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < MI; ++i) af[i] = *(const f16x8*)&As[buf][32 * MI * wm + 32 * i + (lane & 31)][kc];
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[j] = *(const f16x8*)&Bs[buf][32 * NI * wn + 32 * j + (lane & 31)][kc];
  };
  // Step kt: x of step kt+1 is loaded at its start and stored to the other buffer
  // after slice 1; the fragments of slice ks+1 are read before the MFMAs of slice ks.
  // Slice 3's MFMAs straddle the barrier: half are issued before it, then the next
  // step's slice-0 fragments are read, then the other half run while they arrive.
  // nb: the super-block holding step kt+1's pair np.
  f16x8 af[2][MI], bf[2][NI];
  auto mfmas = [&](int f, int t0, int t1) {   // tiles t0 .. t1-1 (t = i*NI + j)
#pragma unroll
    for (int t = t0; t < t1; ++t)
      acc[t / NI][t % NI] =
          __builtin_amdgcn_mfma_f32_32x32x16_f16(af[f][t / NI], bf[f][t % NI], acc[t / NI][t % NI], 0, 0, 0);
  };
  auto step = [&](int kt, const Blk& nb, int np) {
    const int cur = kt & 1;
    float s[2], c[2];
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) {
      frags(cur, ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
      // keep the reads of slice ks+1 ahead of slice ks's MFMAs (the scheduler would
      // otherwise sink them next to their use to save registers)
      __builtin_amdgcn_sched_barrier(0);
      if (ks == 0) {                       // interleaved with slice 0's MFMAs
        scales(nb, np, s, c);
        xload(kt + 1);
      }
      mfmas(ks & 1, 0, MI * NI);
      deq(nb, np, ks, s, c, cur ^ 1);
      if (ks == 1) {
#pragma unroll
        for (int i = 0; i < AC; ++i) *(u32x4*)&As[cur ^ 1][arow[i]][acol[i]] = xs[i];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    mfmas(1, 0, MI * NI / 2);
    deq(nb, np, 3, s, c, cur ^ 1);
    lds_barrier();
    frags(cur ^ 1, 0, af[0], bf[0]);       // past the last step: unused, in bounds
    __builtin_amdgcn_sched_barrier(0);
    mfmas(1, MI * NI / 2, MI * NI);
    __builtin_amdgcn_sched_barrier(0);
  };

  Blk b0, b1;
  bload(0, b0);
  bload(1, b1);
  xload(0);
  {
    float s[2], c[2];
    scales(b0, 0, s, c);
#pragma unroll
    for (int j = 0; j < 4; ++j) deq(b0, 0, j, s, c, 0);
#pragma unroll
    for (int i = 0; i < AC; ++i) *(u32x4*)&As[0][arow[i]][acol[i]] = xs[i];
  }
  lds_barrier();
  frags(0, 0, af[0], bf[0]);
  // super-blocks in pairs: steps 4S..4S+3 use b0 (pairs 1..3 of S) then b1 (pair 0
  // of S+1); b0 is reloaded with S+2 once its last pair has been dequantised
  const int SB = KT / 4;
  int S = 0;
  for (; S + 1 < SB; S += 2) {
    const int kt = 4 * S;
    step(kt, b0, 1);
    step(kt + 1, b0, 2);
    step(kt + 2, b0, 3);
    bload(S + 2, b0);
    step(kt + 3, b1, 0);
    step(kt + 4, b1, 1);
    step(kt + 5, b1, 2);
    step(kt + 6, b1, 3);
    bload(S + 3, b1);
    step(kt + 7, b0, 0);
  }
  if (S < SB) {                            // last super-block (odd count)
    const int kt = 4 * S;
    step(kt, b0, 1);
    step(kt + 1, b0, 2);
    step(kt + 2, b0, 3);
    step(kt + 3, b1, 0);                   // dequantises garbage into an unused buffer
  }
  // D[i][j] of a tile: j = lane%32 (weight row), i = 8(t/4) + 4(lane/32) + t%4 (x row)
  constexpr uint32_t esz = sizeof(YT);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)y, (short)0, (int)((uint32_t)M * (uint32_t)N * esz), ALLOY_RSRC_DW3);
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int n = n0 + 32 * NI * wn + 32 * j + (lane & 31);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int m = m0 + 32 * MI * wm + 32 * i + 8 * (t >> 2) + 4 * (lane >> 5) + (t & 3);
        const uint32_t off = n < N ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * esz : 0x80000000u;
        const float v = acc[i][j][t];      // element copied out before the bit cast
        if constexpr (sizeof(YT) == 4)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr, off, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16)v), yr, off, 0, 0);
      }
    }
}

// kind 0: 256 x 256 tile, kind 1: 256 x 128.  The caller has checked that every
// buffer offset fits 32 bits, that K % 256 == 0 and (nsb > 0) that ws holds the splits.
hipError_t launch_gemm_q4k_w4(int kind, const QArgs& a, const f16* x, int M, void* y, bool y_f32, int N,
                              int splits, int nsb, hipStream_t st) {
  auto go = [&](auto mi, auto ni) {
    constexpr int MI = decltype(mi)::value, NI = decltype(ni)::value;
    const dim3 grid((unsigned)((N + 64 * NI - 1) / (64 * NI)), (unsigned)((M + 64 * MI - 1) / (64 * MI)),
                    (unsigned)splits);
    const int remap = splits == 1 && (grid.x * grid.y) % 8 == 0;
    if (y_f32)
      hipLaunchKernelGGL((k_gemm_q4k_w4<MI, NI, float>), grid, dim3(256), 0, st, a, x, M, (float*)y, N, nsb,
                         remap);
    else
      hipLaunchKernelGGL((k_gemm_q4k_w4<MI, NI, f16>), grid, dim3(256), 0, st, a, x, M, (f16*)y, N, nsb, remap);
    return hipGetLastError();
  };
  if (kind == 1) return go(std::integral_constant<int, 4>(), std::integral_constant<int, 2>());
  return go(std::integral_constant<int, 4>(), std::integral_constant<int, 4>());
}

}  // namespace alloy
