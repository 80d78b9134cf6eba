// Prefill GEMM on MFMA for gfx950: y[M,N] = x[M,K] (fp16) . dequant(w)[N,K]^T with
// the weight tiles dequantised to fp16 in LDS and v_mfma_f32_32x32x16_f16 (fp32
// accumulation).  The Q4_K kernel (k_gemm_q4k) is the prefill hot path; k_gemm serves
// the other formats.  All launched on the caller's HIP stream, no allocation.
#include <type_traits>

#include "gemv.h"
#include "launch.h"
#include "xs.h"

namespace alloy {

// Raw buffer loads with an SGPR offset: the hardware range check covers only the
// VGPR offset (plus the instruction offset), so a load whose VGPR offset is in
// bounds can reach past the buffer through its SGPR offset.  Prefetches that may run
// past the end of the data therefore replace their VGPR offset by kOOB (always out
// of range: such a load reads zero and touches no memory); every buffer below is
// smaller than 2^31 bytes (checked on the host).
constexpr uint32_t kOOB = 0x80000000u;

// ------------------------------------------------------------------ generic prefill GEMM
// Tile 128 (x rows) x 128 (weight rows) x 64 (K), 4 waves as 2x2, each 64x64 from
// 2x2 v_mfma_f32_32x32x16_f16.  The weight tile is dequantised (exact fp32 -> RN fp16)
// into LDS; x is copied as fp16.  Double-buffered: the next step's x and weight
// elements are decoded into registers before the current step's MFMAs and stored to
// the other buffer after them, one barrier per step.
constexpr int GBM = 128, GBN = 128, GBK = 64, GLD = GBK + 8;

template <class F, typename XT>
__global__ __launch_bounds__(256) void k_gemm(QArgs a, const XT* x, int M, void* y, int y_f32,
                                              int64_t N) {
  __shared__ __attribute__((aligned(16))) f16 As[2][GBM][GLD];
  __shared__ __attribute__((aligned(16))) f16 Bs[2][GBN][GLD];
  const int K = a.K;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * GBM;
  const int64_t n0 = (int64_t)blockIdx.x * GBN;
  f32x16 acc[2][2];
#pragma unroll
  for (int tm = 0; tm < 2; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[tm][tn][e] = 0.f;

  // this thread's share of a step: x rows tid/8 + 32c, 8 halves at column 8*(tid%8);
  // weight row tid/2, elements 32*(tid%2) .. +31
  const int brow = tid >> 1, bk = (tid & 1) * 32;
  f16x8 xv[4], wv[4];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c, row = idx >> 3, col = (idx & 7) * 8;
      const int64_t gm = m0 + row;
      xv[c] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      if (gm < M && k0 + col < K) xv[c] = ld_x8<XT>(x + gm * K + k0 + col);
    }
    const int64_t gn = n0 + brow;
    if (gn < N && k0 + bk < K) dec32_f16<F>(a, gn, k0 + bk, wv);
    else {
#pragma unroll
      for (int j = 0; j < 4; ++j) wv[j] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int idx = tid + 256 * c;
      *(f16x8*)&As[buf][idx >> 3][(idx & 7) * 8] = xv[c];
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) *(f16x8*)&Bs[buf][brow][bk + 8 * j] = wv[j];
  };

  fetch(0);
  put(0);
  __syncthreads();
  for (int k0 = 0, cur = 0; k0 < K; k0 += GBK, cur ^= 1) {
    const bool more = k0 + GBK < K;
    if (more) fetch(k0 + GBK);
#pragma unroll
    for (int ks = 0; ks < GBK; ks += 16) {
      f16x8 af[2], bf[2];
      const int kc = ks + 8 * (lane >> 5);
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        af[t] = *(const f16x8*)&As[cur][64 * wm + 32 * t + (lane & 31)][kc];
        bf[t] = *(const f16x8*)&Bs[cur][64 * wn + 32 * t + (lane & 31)][kc];
      }
#pragma unroll
      for (int tm = 0; tm < 2; ++tm)
#pragma unroll
        for (int tn = 0; tn < 2; ++tn)
          acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[tm], bf[tn], acc[tm][tn], 0, 0, 0);
    }
    if (more) put(cur ^ 1);
    __syncthreads();
  }
  // D[i][j]: j = lane%32 (weight row), i = 8(t/4) + 4(lane/32) + t%4 (x row)
#pragma unroll
  for (int tm = 0; tm < 2; ++tm)
#pragma unroll
    for (int tn = 0; tn < 2; ++tn) {
      const int64_t gn = n0 + 64 * wn + 32 * tn + (lane & 31);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int64_t gm = m0 + 64 * wm + 32 * tm + 8 * (t >> 2) + 4 * (lane >> 5) + (t & 3);
        if (gm < M && gn < N) store_y(y, y_f32, gm * N + gn, acc[tm][tn][t]);
      }
    }
}

// ------------------------------------------------------------------ Q4_K prefill GEMM
// 512 threads = 8 waves as 2 (x rows) x 4 (weight rows); wave tile 32*MI x 32*NI of
// v_mfma_f32_32x32x16_f16 tiles, workgroup tile QBM = 64*MI x QBN = 128*NI; K advances
// in steps of 64 (one super-block pair), one barrier per step.  x rows past M and
// weight rows past N read as zero (out-of-range buffer offsets); stores past them are
// dropped.  Weight dequant: a nibble masked into one half of a dword is the fp16
// denormal q*2^-24 (16q*2^-24 for a high nibble), and v_fma_mix with the scale
// d*sc*2^24 (2^20 high) and offset -dmin*m gives the exact fp32 weight d*sc*q - dmin*m
// (every product is exact in fp32: one rounding), rounded to fp16 (RNE).
//  * LDS rows of 128 bytes (64 halves) without padding; 16-byte chunk c of row r sits
//    at chunk c ^ swz(r), swz(r) = (r & 7) ^ ((r >> 3) & 1), so the 16 lanes of every
//    b128 LDS pass (64 banks) touch 16 consecutive rows at one logical chunk and never
//    share a bank, for the MFMA operand reads and for the dequant stores alike;
//  * x copied global -> LDS by the buffer unit (buffer_load_dwordx4 ... lds: lane l of
//    an instruction writes bytes 16l .. 16l+15 of a 1 KB LDS range), two steps ahead
//    through three x stages, with no VGPR staging;
//  * one nibble per thread: TPR = 512/QBN threads share a weight row, thread half h
//    takes the low (h = 0: sub-block 2p, elements 0..31 of the step) or high (h = 1:
//    sub-block 2p+1, elements 32..63) nibbles of its byte range, so it needs one
//    scale and writes whole 16-byte chunks of consecutive rows;
//  * raw weight bytes loaded three steps ahead into a ring of three pair slots (and
//    super-block headers into a ring of three), MFMA operand fragments read one K
//    substep ahead.
// Loads retire in order, so at the end of step kt one s_waitcnt on the number of
// loads issued after x(kt+1) completes that copy while x(kt+2) and the weight
// prefetches stay in flight.  The step barrier is the bare s_barrier with that wait
// and lgkmcnt(0) (the dequant stores) made explicit: a workgroup fence would also
// wait for x(kt+2).  Scheduling barriers on both sides keep every LDS access on
// its side of it.  Each stage is its own LDS array and the step loop is
// unrolled over 12 steps (3 x stages, 2 weight stages, 3 pair slots, 3 headers), so
// every index is a compile-time constant and the compiler's own wait for an x copy
// never covers reads of another stage.
__device__ __forceinline__ int lds_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }
// buffer_load_dwordx4 ... lds: 16 bytes per lane from buffer offset vo + so to LDS
// address lds + 16 * lane (lds is wave-uniform)
__device__ __forceinline__ void lds_copy16(__amdgpu_buffer_rsrc_t r, uint8_t* lds, uint32_t vo, uint32_t so) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, vo, so, 0, 0);
}
// s_waitcnt immediate: vmcnt(n) (n < 64), no wait on the export counter, lgkmcnt(l)
constexpr int waitcnt_enc(int n, int l) { return 0x0070 | (l << 8) | (n & 15) | ((n >> 4) << 14); }
// workgroup barrier of the swizzled GEMM: this wave's loads but the last n and all
// its LDS accesses complete, then s_barrier, with no instruction moved across
template <int N>
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_s_waitcnt(waitcnt_enc(N, 0));
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// fp16 pair (RN16(f(a)), RN16(f(b))) with f(h) = h * s + c for the low (or high) fp16 halves
// of v0 and v1
__device__ __forceinline__ uint32_t q4k_pair(uint32_t v0, uint32_t v1, bool hi_half, float s, float c) {
  const f16x2 a = __builtin_bit_cast(f16x2, v0), b = __builtin_bit_cast(f16x2, v1);
  const f16 ha = hi_half ? a[1] : a[0], hb = hi_half ? b[1] : b[0];
  const float fa = __builtin_fmaf((float)ha, s, c), fb = __builtin_fmaf((float)hb, s, c);
  return __builtin_bit_cast(uint32_t, f16x2{(f16)fa, (f16)fb});
}

template <int MI, int NI, typename YT>
__global__ __launch_bounds__(512) void k_gemm_q4k(QArgs a, const f16* x, int M, YT* y, int N, int nsb) {
  constexpr int QBM = 64 * MI, QBN = 128 * NI;
  constexpr int TPR = 512 / QBN;                  // threads per weight row: 2 (QBN 256) or 4
  constexpr int BPT = 64 / TPR;                   // quant bytes of a pair per thread: 32 or 16
  constexpr int CPT = BPT / 8;                    // 8-element chunks written per step: 4 or 2
  constexpr int LPT = BPT / 16;                   // 16-byte raw loads per step: 2 or 1
  __shared__ __attribute__((aligned(1024))) uint8_t xs0[QBM * 128], xs1[QBM * 128], xs2[QBM * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t ws0[QBN * 128], ws1[QBN * 128];
  uint8_t* const XS[3] = {xs0, xs1, xs2};
  uint8_t* const WS[2] = {ws0, ws1};
  const int K = a.K, KT = nsb > 0 ? 4 * nsb : K / 64, SB = KT / 4;
  const uint32_t kb = nsb > 0 ? (uint32_t)blockIdx.z * (uint32_t)nsb : 0u;
  if (nsb > 0) y += (size_t)blockIdx.z * (size_t)M * (size_t)N;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 2, wn = wave & 3;
  const int m0 = (int)blockIdx.y * QBM, n0 = (int)blockIdx.x * QBN;
  const uint32_t rb = (uint32_t)a.rb;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), ALLOY_RSRC_DW3);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.w, (short)0, (int)((uint32_t)N * rb), ALLOY_RSRC_DW3);

  // x copy: wave w's instruction i fills rows R0 = 8(MI*w + i) .. R0+7 of the stage;
  // lane l lands in row R0 + l/8, physical chunk l%8, i.e. logical chunk (l%8)^swz.
  uint32_t xoff[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int r = 8 * (MI * wave + i) + (lane >> 3), c = (lane & 7) ^ lds_swz(r);
    xoff[i] = ((uint32_t)(m0 + r) * (uint32_t)K + 256u * kb + 8u * (uint32_t)c) * 2u;
  }
  auto xcopy = [&](int kt, uint8_t* st) {       // MI loads; past the range: zeros
    const uint32_t so = 128u * (uint32_t)kt;
#pragma unroll
    for (int i = 0; i < MI; ++i) lds_copy16(xr, st + 1024 * (MI * wave + i), kt < KT ? xoff[i] : kOOB, so);
  };

  // weight rows: thread -> row br, nibble half h, byte part
  const int br = tid % QBN, q = tid / QBN, h = q & 1, part = q >> 1;
  const uint32_t wrow = (uint32_t)(n0 + br) * rb + 144u * kb;
  const uint32_t qoff = wrow + 16u + (uint32_t)(BPT * part);
  const uint32_t m_nib = h ? 0x00F000F0u : 0x000F000Fu;
  const float smul = h ? 1048576.f : 16777216.f;      // 2^20 (high nibbles hold 16q) or 2^24
  const int swb = lds_swz(br);
  const int c0 = 4 * h + (BPT / 8) * part;            // first logical chunk this thread writes
  u32x4 raw[3][LPT];                                  // pair slots (pair index mod 3)
  u32x4 hdr[3];                                       // super-block headers (index mod 3)
  auto rload = [&](int pair, u32x4 (&slot)[LPT]) {    // LPT loads
    const int sbi = pair >> 2;
    const uint32_t so = (uint32_t)sbi * 144u + 32u * (uint32_t)(pair & 3);
    const uint32_t vo = sbi < SB ? qoff : kOOB;
#pragma unroll
    for (int e = 0; e < LPT; ++e) slot[e] = __builtin_amdgcn_raw_buffer_load_b128(wr, vo + 16u * e, so, 0);
  };
  auto hload = [&](int sbi, u32x4& hd) {              // one load
    hd = __builtin_amdgcn_raw_buffer_load_b128(wr, sbi < SB ? wrow : kOOB, (uint32_t)sbi * 144u, 0);
  };
  // scale / offset of this thread's sub-block 2p+h
  auto scale = [&](const u32x4& hd, int p, float& s, float& c) {
    uint32_t sc, mn;
    q4k_scale_min(hd.y, hd.z, hd.w, 2 * p + h, sc, mn);
    s = h2f(hd.x) * (float)sc * smul;
    c = -(h2f(hd.x >> 16) * (float)mn);
  };
  // chunk j (8 elements) of this thread's share of a pair: dwords 2j, 2j+1 of its bytes
  auto deq = [&](const u32x4 (&slot)[LPT], int j, float s, float c, uint8_t* st) {
    const u32x4& v = slot[j >> 1];
    const uint32_t w0 = (j & 1) ? v.z : v.x, w1 = (j & 1) ? v.w : v.y;
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t w = e ? w1 : w0;
      const uint32_t ea = w & m_nib, eb = (w >> 8) & m_nib;     // bytes (0, 2), (1, 3)
      o[2 * e] = q4k_pair(ea, eb, false, s, c);
      o[2 * e + 1] = q4k_pair(ea, eb, true, s, c);
    }
    *(u32x4*)(st + br * 128 + (((c0 + j) ^ swb) << 4)) = u32x4{o[0], o[1], o[2], o[3]};
  };

  // MFMA operand fragments: lane row l%32 of each 32-row tile, logical chunk
  // 2ks + l/32; the swizzle of rows 32t + l%32 is that of l%32
  // (row bits 7.., chunk bits 4..6: the substep's chunk 2ks + l/32 swizzled is
  // that of substep 0 with ks XORed into bits 5..6)
  const uint32_t foff0 = (uint32_t)((lane & 31) * 128 + (((lane >> 5) ^ lds_swz(lane & 31)) << 4));
  const int arow = 32 * MI * wm, brow = 32 * NI * wn;
  f16x8 af[2][MI], bf[2][NI];
  auto frag = [&](const uint8_t* xsb, const uint8_t* wsb, int ks, int s) {
    const uint32_t fo = foff0 ^ ((uint32_t)ks << 5);
#pragma unroll
    for (int i = 0; i < MI; ++i) af[s][i] = *(const f16x8*)(xsb + (arow + 32 * i) * 128 + fo);
#pragma unroll
    for (int j = 0; j < NI; ++j) bf[s][j] = *(const f16x8*)(wsb + (brow + 32 * j) * 128 + fo);
  };

  f32x16 acc[MI][NI];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NI; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // step kt (J = kt % 12, a compile-time constant): MFMAs on x stage kt%3 and weight
  // stage kt%2; x(kt+2) copied into stage (kt+2)%3 first; pair kt+1 (slot (kt+1)%3,
  // header of super-block (kt+1)/4 in the slot of its parity) dequantised into weight
  // stage (kt+1)%2; pair kt+4 loaded into the freed slot last (and, when it starts a
  // super-block, that super-block's header).
  auto step = [&](auto Jc, int kt) {
    constexpr int J = decltype(Jc)::value;
    constexpr int P1 = (J + 1) & 3, R1 = (J + 1) % 3;            // pair within its super-block, ring slot
    constexpr int H1 = ((J + 1) >> 2) % 3, HN = ((J >> 2) + 1) % 3;  // header of pair kt+1 / loaded now
    constexpr bool hnow = (J & 3) == 0, hprev = (J & 3) == 1;  // header loads at this / the previous step
    const uint8_t* xc = XS[J % 3];
    const uint8_t* wc = WS[J & 1];
    xcopy(kt + 2, XS[(J + 2) % 3]);
    float s, c;
    scale(hdr[H1], P1, s, c);
    frag(xc, wc, 0, 0);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int cs = ks & 1;
      if (ks < 3) frag(xc, wc, ks + 1, cs ^ 1);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int jn = 0; jn < NI; ++jn)
          acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cs][i], bf[cs][jn], acc[i][jn], 0, 0, 0);
      if (CPT == 4 || (ks & 1) == 0) deq(raw[R1], CPT == 4 ? ks : ks >> 1, s, c, WS[(J + 1) & 1]);
    }
    // the prefetch loads stay behind this step's x copy (the wait below counts on it)
    __builtin_amdgcn_sched_barrier(0);
    rload(kt + 4, raw[R1]);
    if constexpr (hnow) hload((kt >> 2) + 1, hdr[HN]);   // its slot's last use: super-block kt/4 - 2
    // x(kt+1), copied at the top of step kt-1, is done once at most the loads issued
    // after it are outstanding: the prefetch of step kt-1, x(kt+2) and this prefetch
    step_barrier<2 * LPT + MI + (hnow ? 1 : 0) + (hprev ? 1 : 0)>();
  };

  // prologue: header 0; pairs 0..2 (slots 0..2); x of steps 0 and 1; pair 0
  // dequantised into weight stage 0; pair 3 into slot 0 (the loop's step-(-1) prefetch)
  hload(0, hdr[0]);
#pragma unroll
  for (int p = 0; p < 3; ++p) rload(p, raw[p]);
  xcopy(0, xs0);
  xcopy(1, xs1);
  {
    float s, c;
    scale(hdr[0], 0, s, c);
#pragma unroll
    for (int j = 0; j < CPT; ++j) deq(raw[0], j, s, c, ws0);
  }
  __builtin_amdgcn_sched_barrier(0);
  rload(3, raw[0]);
  step_barrier<MI + LPT>();                          // x(0) done: x(1) and pair 3 may be in flight
  // twelve steps (three super-blocks) per iteration, then 0, 4 or 8 more
  int kt = 0;
  for (; kt + 12 <= KT; kt += 12) {
    step(std::integral_constant<int, 0>(), kt + 0);
    step(std::integral_constant<int, 1>(), kt + 1);
    step(std::integral_constant<int, 2>(), kt + 2);
    step(std::integral_constant<int, 3>(), kt + 3);
    step(std::integral_constant<int, 4>(), kt + 4);
    step(std::integral_constant<int, 5>(), kt + 5);
    step(std::integral_constant<int, 6>(), kt + 6);
    step(std::integral_constant<int, 7>(), kt + 7);
    step(std::integral_constant<int, 8>(), kt + 8);
    step(std::integral_constant<int, 9>(), kt + 9);
    step(std::integral_constant<int, 10>(), kt + 10);
    step(std::integral_constant<int, 11>(), kt + 11);
  }
  if (kt + 4 <= KT) {
    step(std::integral_constant<int, 0>(), kt + 0);
    step(std::integral_constant<int, 1>(), kt + 1);
    step(std::integral_constant<int, 2>(), kt + 2);
    step(std::integral_constant<int, 3>(), kt + 3);
    if (kt + 8 <= KT) {
      step(std::integral_constant<int, 4>(), kt + 4);
      step(std::integral_constant<int, 5>(), kt + 5);
      step(std::integral_constant<int, 6>(), kt + 6);
      step(std::integral_constant<int, 7>(), kt + 7);
    }
  }
  // D[i][j] of a tile: j = lane%32 (weight row), i = 8(t/4) + 4(lane/32) + t%4 (x row)
  constexpr uint32_t esz = sizeof(YT);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)y, (short)0, (int)((uint32_t)M * (uint32_t)N * esz), ALLOY_RSRC_DW3);
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int jn = 0; jn < NI; ++jn) {
      const int n = n0 + brow + 32 * jn + (lane & 31);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int m = m0 + arow + 32 * i + 8 * (t >> 2) + 4 * (lane >> 5) + (t & 3);
        const uint32_t off = n < N ? ((uint32_t)m * (uint32_t)N + (uint32_t)n) * esz : kOOB;
        const float v = acc[i][jn][t];
        if constexpr (sizeof(YT) == 4)
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), yr, off, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16)v), yr, off, 0, 0);
      }
    }
}

// Sum of the S fp32 split-K partial slices, in slice order (deterministic).
template <typename YT>
__global__ __launch_bounds__(256) void k_splitk_sum(const float* ws, int S, int64_t mn, YT* y) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  f32x4 acc = *(const f32x4*)(ws + i);
  for (int z = 1; z < S; ++z) acc += *(const f32x4*)(ws + (int64_t)z * mn + i);
  if constexpr (sizeof(YT) == 4) {
    *(f32x4*)((float*)y + i) = acc;
  } else {
    const float a0 = acc[0], a1 = acc[1], a2 = acc[2], a3 = acc[3];   // elements copied out first
    *(f16x4*)((f16*)y + i) = f16x4{(f16)a0, (f16)a1, (f16)a2, (f16)a3};
  }
}

// Q4_K GEMM plan: tile kind (0 = 256x256, 1 = 128x256, 2 = 128x128, 3 = 64x256,
// 4 = 64x128) and K splits S.  Each kind's measured full-chip rate (TFLOP/s on
// MI355X) is scaled by the fraction of CU slots its tile count x S fills in the last
// round of workgroups; a split adds the partial-sum pass ((S+1) fp32 M x N tiles of
// HBM traffic) and one launch.  S divides the super-blocks, at least two per split.
struct GemmPlan { int kind, splits; };
static GemmPlan gemm_plan(int64_t M, int64_t N, int64_t K, bool allow_split) {
  const int cus = cu_count();
  const int bm[5] = {256, 128, 128, 64, 64}, bn[5] = {256, 256, 128, 256, 128};
  const double rate[5] = {1000e12, 790e12, 600e12, 590e12, 420e12};
  const double flops = 2.0 * (double)M * (double)N * (double)K;
  const int64_t sb = K / 256;
  GemmPlan best{0, 1};
  double best_t = 1e30;
  for (int k = 0; k < 5; ++k) {
    const int64_t tl = ((M + bm[k] - 1) / bm[k]) * ((N + bn[k] - 1) / bn[k]);
    for (int S = 1; S <= (allow_split ? 4 : 1); ++S) {
      if (S > 1 && (sb % S || sb / S < 2)) continue;
      const int64_t wg = tl * S, rounds = (wg + cus - 1) / cus;
      double t = flops / (rate[k] * (double)wg / (double)(rounds * cus));
      if (S > 1) t += (double)(S + 1) * (double)M * (double)N * 4.0 / 5e12 + 2e-6;
      if (t < best_t) { best_t = t; best = GemmPlan{k, S}; }
    }
  }
  return best;
}

static bool gemm_q4k_fits(int64_t M, int64_t N, const QArgs& a) {   // 32-bit buffer offsets
  return (uint64_t)M * (uint64_t)a.K * 2u < (1ull << 31) && (uint64_t)N * (uint64_t)a.rb < (1ull << 31) &&
         (uint64_t)M * (uint64_t)N * 4u < (1ull << 31);
}

int64_t gemm_workspace_bytes(int fmt, int64_t M, int64_t N, int64_t K) {
  if (fmt != F_Q4_K || M <= 64 || K % 256) return 0;
  const GemmPlan p = gemm_plan(M, N, K, true);
  return p.splits > 1 ? (int64_t)p.splits * M * N * 4 : 0;
}

static hipError_t launch_gemm_q4k(const QArgs& a, const void* x, void* y, bool y_f32, int64_t M, int64_t N,
                                  const Opts& o, void* ws, int64_t ws_bytes, hipStream_t st) {
  GemmPlan p = o.variant >= 4 ? GemmPlan{o.variant - 4, 1} : gemm_plan(M, N, a.K, ws != nullptr);
  if (o.variant >= 4 && o.splits > 1 && (a.K / 256) % o.splits == 0 && a.K / 256 / o.splits >= 2)
    p.splits = o.splits;             // forced split (falls back to none without the workspace)
  if (p.splits > 1 &&
      (ws_bytes < (int64_t)p.splits * M * N * 4 || ((uintptr_t)ws & 15) || ((uintptr_t)y & 15) || (M * N) % 4))
    p = o.variant >= 4 ? GemmPlan{p.kind, 1} : gemm_plan(M, N, a.K, false);
  const int nsb = p.splits > 1 ? (int)(a.K / 256 / p.splits) : 0;
  auto sum_splits = [&]() {
    const int64_t mn = M * N, blocks = (mn / 4 + 255) / 256;
    if (y_f32)
      hipLaunchKernelGGL(k_splitk_sum<float>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)ws, p.splits,
                         mn, (float*)y);
    else
      hipLaunchKernelGGL(k_splitk_sum<f16>, dim3((unsigned)blocks), dim3(256), 0, st, (const float*)ws, p.splits,
                         mn, (f16*)y);
    return hipGetLastError();
  };
  auto go = [&](auto mi, auto ni) {
    constexpr int MI = decltype(mi)::value, NI = decltype(ni)::value;
    const dim3 grid((unsigned)((N + 128 * NI - 1) / (128 * NI)), (unsigned)((M + 64 * MI - 1) / (64 * MI)),
                    (unsigned)p.splits);
    if (p.splits > 1)
      hipLaunchKernelGGL((k_gemm_q4k<MI, NI, float>), grid, dim3(512), 0, st, a, (const f16*)x, (int)M, (float*)ws,
                         (int)N, nsb);
    else if (y_f32)
      hipLaunchKernelGGL((k_gemm_q4k<MI, NI, float>), grid, dim3(512), 0, st, a, (const f16*)x, (int)M, (float*)y,
                         (int)N, 0);
    else
      hipLaunchKernelGGL((k_gemm_q4k<MI, NI, f16>), grid, dim3(512), 0, st, a, (const f16*)x, (int)M, (f16*)y,
                         (int)N, 0);
    hipError_t e = hipGetLastError();
    return e != hipSuccess || p.splits == 1 ? e : sum_splits();
  };
  switch (p.kind) {
    case 0: return go(std::integral_constant<int, 4>(), std::integral_constant<int, 2>());
    case 1: return go(std::integral_constant<int, 2>(), std::integral_constant<int, 2>());
    case 3: return go(std::integral_constant<int, 1>(), std::integral_constant<int, 2>());
    case 4: return go(std::integral_constant<int, 1>(), std::integral_constant<int, 1>());
    default: return go(std::integral_constant<int, 2>(), std::integral_constant<int, 1>());
  }
}

template <class F>
static hipError_t launch_gemm_generic(const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32, int64_t M,
                                      int64_t N, hipStream_t st) {
  dim3 grid((unsigned)((N + GBN - 1) / GBN), (unsigned)((M + GBM - 1) / GBM));
  if (x_f32)
    hipLaunchKernelGGL((k_gemm<F, float>), grid, dim3(256), 0, st, a, (const float*)x, (int)M, y, (int)y_f32, N);
  else
    hipLaunchKernelGGL((k_gemm<F, f16>), grid, dim3(256), 0, st, a, (const f16*)x, (int)M, y, (int)y_f32, N);
  return hipGetLastError();
}

hipError_t launch_gemm(int fmt, const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32,
                       int64_t M, int64_t N, const Opts& o, void* ws, int64_t ws_bytes, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  if (fmt == F_Q4_K && !x_f32 && gemm_q4k_fits(M, N, a) && (M > 64 || o.variant >= 4) && o.variant != 1)
    return launch_gemm_q4k(a, x, y, y_f32, M, N, o, ws, ws_bytes, st);
  switch (fmt) {
    case F_Q8_0: return launch_gemm_generic<FQ80>(a, x, x_f32, y, y_f32, M, N, st);
    case F_Q5_0: return launch_gemm_generic<FQ50>(a, x, x_f32, y, y_f32, M, N, st);
    case F_Q4_K: return launch_gemm_generic<FQ4K>(a, x, x_f32, y, y_f32, M, N, st);
    case F_Q6_K: return launch_gemm_generic<FQ6K>(a, x, x_f32, y, y_f32, M, N, st);
    case F_MLX: return launch_gemm_generic<FMLX>(a, x, x_f32, y, y_f32, M, N, st);
    case F_Q8_0S: return launch_gemm_generic<FQ80S>(a, x, x_f32, y, y_f32, M, N, st);
    case F_Q5_0S: return launch_gemm_generic<FQ50S>(a, x, x_f32, y, y_f32, M, N, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace alloy
