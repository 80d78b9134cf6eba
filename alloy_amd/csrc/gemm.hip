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
// Workgroup barrier of the swizzled GEMMs: this wave's loads but the last n and all
// its LDS accesses complete, then s_barrier, with no instruction moved across.  The
// GEMMs use n = 0.  A partial count (only the loads issued after a stage's
// buffer-to-LDS copy outstanding) assumes that the copies and the plain loads retire
// in issue order; with it the 4096 x 14336 x 4096 Q4_K product differed between
// repeated runs (60 of 400), with the full wait in none of 400.
template <int N>
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_s_waitcnt(waitcnt_enc(N, 0));
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
}
// the same with LDS accesses only (loads stay in flight)
__device__ __forceinline__ void step_barrier_lds() {
  __builtin_amdgcn_s_waitcnt(waitcnt_enc(63, 0));
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
  u32x4 raw[4][LPT];                                  // pair slots (pair index mod 4)
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
  // stage kt%2; first x(kt+2) copied into stage (kt+2)%3 and pair kt+4 loaded into
  // ring slot kt%4 (its pair kt was consumed by the previous step; and, when it
  // starts a super-block, that super-block's header), so they have the whole step to
  // land before the closing full wait; pair kt+1 (slot (kt+1)%4, header of
  // super-block (kt+1)/4) dequantised into weight stage (kt+1)%2.
  auto step = [&](auto Jc, int kt) {
    constexpr int J = decltype(Jc)::value;
    constexpr int P1 = (J + 1) & 3, R1 = (J + 1) & 3, RN = J & 3;   // pair within its super-block, ring slots
    constexpr int H1 = ((J + 1) >> 2) % 3, HN = ((J >> 2) + 1) % 3;  // header of pair kt+1 / loaded now
    constexpr bool hnow = (J & 3) == 0;                        // a header load at this step
    const uint8_t* xc = XS[J % 3];
    const uint8_t* wc = WS[J & 1];
    xcopy(kt + 2, XS[(J + 2) % 3]);
    rload(kt + 4, raw[RN]);
    if constexpr (hnow) hload((kt >> 2) + 1, hdr[HN]);   // its slot's last use: super-block kt/4 - 2
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
    __builtin_amdgcn_sched_barrier(0);
    // every load lands before a full wait at the end of every even step, so each has
    // one or two steps: x(k) (issued at step k-2) is needed at step k, pair p (step
    // p-4) at step p-1, a header (step 4s-4) at step 4s-1; odd steps order the LDS
    // stages only
    if constexpr ((J & 1) == 0) step_barrier<0>();
    else step_barrier_lds();
  };

  // prologue: header 0; pairs 0..3 (slots 0..3); x of steps 0 and 1; pair 0
  // dequantised into weight stage 0
  hload(0, hdr[0]);
#pragma unroll
  for (int p = 0; p < 4; ++p) rload(p, raw[p]);
  xcopy(0, xs0);
  xcopy(1, xs1);
  {
    float s, c;
    scale(hdr[0], 0, s, c);
#pragma unroll
    for (int j = 0; j < CPT; ++j) deq(raw[0], j, s, c, ws0);
  }
  __builtin_amdgcn_sched_barrier(0);
  step_barrier<0>();
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

// ------------------------------------------------------------------ other formats' prefill GEMM
// The Q4_K kernel's structure (swizzled unpadded LDS tiles, x copied to LDS by the
// buffer unit two steps ahead through three stages, raw weight bytes in a three-slot
// register ring three steps ahead, one barrier per 64-element K step) with the weight
// bytes read and decoded by a per-format provider W.  Weight tile rows are 256 wide
// (QBN = 256): thread tid serves row tid % 256 and elements 32 h .. 32 h + 31 of each
// step, h = tid / 256 (uniform per wave), and writes them as four 16-byte chunks.
//   W::NL                  loads per step and thread (issued whatever the data, so
//                          the barrier's load count is a constant)
//   W::Raw, W::load(s, r, kt, h, valid, raw)   the bytes of row r for step kt (valid
//                          false: out-of-range offsets, zeros, no traffic)
//   W::decode<CH>(raw, h, o, kt)  chunk CH (elements 8 CH .. 8 CH + 7) of the 32
//                          weights as fp16 (exact value rounded once), o[i] = elements
//                          8 CH + 2i, + 1
// No load that carries needed bytes reaches past its block: a load that only partly
// fits the buffer reads as zero as a whole.
struct GemmArgs {                  // one matrix: buffers, their byte sizes, per-row strides
  const void *w, *aux, *s, *b;
  uint32_t wbytes, sbytes;         // bytes of w (and aux) / of s and b (0: absent)
  uint32_t rb, sb;                 // bytes per row of w (and aux) / of s and b
};
struct GemmRows {                  // the same as buffer views (built on the device)
  __amdgpu_buffer_rsrc_t w, aux, s, b;
  uint32_t rb, sb;
  __device__ explicit GemmRows(const GemmArgs& g) {
    w = __builtin_amdgcn_make_buffer_rsrc((void*)g.w, (short)0, (int)g.wbytes, ALLOY_RSRC_DW3);
    aux = __builtin_amdgcn_make_buffer_rsrc((void*)g.aux, (short)0, g.aux ? (int)g.wbytes : 0, ALLOY_RSRC_DW3);
    s = __builtin_amdgcn_make_buffer_rsrc((void*)g.s, (short)0, g.s ? (int)g.sbytes : 0, ALLOY_RSRC_DW3);
    b = __builtin_amdgcn_make_buffer_rsrc((void*)g.b, (short)0, g.b ? (int)g.sbytes : 0, ALLOY_RSRC_DW3);
    rb = g.rb;
    sb = g.sb;
  }
};
// two elements as fp16 denormals (integers < 1024 in the halves of v) -> RN16(v * s + c)
__device__ __forceinline__ uint32_t gw_dq2(uint32_t v, float s, float c) { return xs_dq2(v, s, c); }

// Q8_0 wire blocks (34 B: fp16 d | 32 int8): thread h decodes block 2 kt + h of its row
// (rows are 68 K / 64 bytes, so the pair of blocks starts 4-byte aligned).  Block 0 is
// read as 16 + 16 + 2 bytes from its start (quants realigned by 2 bytes), block 1 (2
// bytes past a 4-byte boundary) as d then 16 + 16 aligned quant bytes: the same three
// load sizes at per-thread offsets, all inside the block.
struct GWQ80 {
  static constexpr int NL = 3;
  struct Raw { u32x4 a, b; uint32_t t; };
  __device__ static void load(const GemmRows& s, uint32_t row, int kt, int h, bool valid, Raw& r) {
    const uint32_t bo = valid ? row * s.rb + 68u * (uint32_t)kt + 34u * (uint32_t)h : kOOB;
    r.a = bld16(s.w, bo + (h ? 2u : 0u));
    r.b = bld16(s.w, bo + (h ? 18u : 16u));
    r.t = bld2(s.w, bo + (h ? 0u : 32u));
  }
  template <int CH>
  __device__ static void decode(const Raw& r, int h, uint32_t (&o)[4], int) {
    const uint32_t w[9] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.t};
    const float d = h2f(h ? r.t : r.a.x), s = d * 16777216.f, c = -128.f * d;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      // quant bytes 4i .. 4i + 3: block 0 at bytes 2 + 4i of its run, block 1 aligned
      constexpr int i0 = 2 * CH;
      const int i = i0 + k;
      const uint32_t q = (h ? w[i] : __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2)) ^ 0x80808080u;
      o[2 * k] = gw_dq2(__builtin_amdgcn_perm(0u, q, 0x0c010c00u), s, c);
      o[2 * k + 1] = gw_dq2(__builtin_amdgcn_perm(0u, q, 0x0c030c02u), s, c);
    }
  }
};

// Q5_0 wire blocks (22 B: fp16 d | u32 qh | qs[16]): thread h decodes block 2 kt + h
// (rows are 44 K / 64 bytes).  Block 0 (4-byte aligned) is read as 16 + 4 + 2 bytes
// and realigned; block 1 (2 bytes past a boundary) as d, then qh and qs aligned.
struct GWQ50 {
  static constexpr int NL = 3;
  struct Raw { u32x4 a; uint32_t m, t; };
  __device__ static void load(const GemmRows& s, uint32_t row, int kt, int h, bool valid, Raw& r) {
    const uint32_t bo = valid ? row * s.rb + 44u * (uint32_t)kt + 22u * (uint32_t)h : kOOB;
    r.a = bld16(s.w, bo + (h ? 6u : 0u));     // block 1: qs
    r.m = bld4(s.w, bo + (h ? 2u : 16u));     // block 1: qh
    r.t = bld2(s.w, bo + (h ? 0u : 20u));     // block 1: d
  }
  template <int CH>
  __device__ static void decode(const Raw& r, int h, uint32_t (&o)[4], int) {
    const float d = h2f(h ? r.t : r.a.x), s = d * 16777216.f, c = -16.f * d;
    const uint32_t hq = h ? r.m : __builtin_amdgcn_alignbyte(r.a.y, r.a.x, 2);
    const uint32_t qs[4] = {h ? r.a.x : __builtin_amdgcn_alignbyte(r.a.z, r.a.y, 2),
                            h ? r.a.y : __builtin_amdgcn_alignbyte(r.a.w, r.a.z, 2),
                            h ? r.a.z : __builtin_amdgcn_alignbyte(r.m, r.a.w, 2),
                            h ? r.a.w : __builtin_amdgcn_alignbyte(r.t, r.m, 2)};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // elements 2p, 2p + 1 (p = 4 CH + k): low (p < 8) or high nibbles of qs bytes
      // 2p % 16, + 1, and qh bits 2p, 2p + 1 moved to bits 4 and 20
      const int p = 4 * CH + k, e = 2 * p, j = e & 15;
      const uint32_t v = __builtin_amdgcn_perm(0u, qs[j >> 2], (j & 2) ? 0x0c030c02u : 0x0c010c00u) >> (e >= 16 ? 4 : 0);
      const uint32_t hb = (__builtin_amdgcn_ubfe(hq, e, 2) * 0x00080010u) & 0x00100010u;
      o[k] = gw_dq2((v & 0x000F000Fu) | hb, s, c);
    }
  }
};

// MLX 4-bit affine (qweight u8 [N, K/2], 8 nibbles per word, low first; fp16 scales /
// biases [N, K/gs], gs a multiple of 32): thread h's 32 elements are 16 qweight bytes
// of one group
struct GWMLX {
  static constexpr int NL = 3;
  static constexpr double R128 = 0.55;           // 128x256 rate / 256x256 rate (measured)
  struct Raw { u32x4 q; uint32_t s, b; };
  __device__ static void load(const GemmRows& s, uint32_t row, int kt, int h, bool valid, Raw& r, int gs) {
    const uint32_t e0 = 64u * (uint32_t)kt + 32u * (uint32_t)h;
    r.q = bld16(s.w, valid ? row * s.rb + e0 / 2u : kOOB);
    const uint32_t so = valid ? row * s.sb + 2u * (e0 / (uint32_t)gs) : kOOB;
    r.s = bld2(s.s, so);
    r.b = bld2(s.b, so);
  }
  template <int CH>
  __device__ static void decode(const Raw& r, int, uint32_t (&o)[4], int) {
    const float sc = h2f(r.s), s = sc * 16777216.f, c = h2f(r.b);
    const uint32_t v = CH == 0 ? r.q.x : CH == 1 ? r.q.y : CH == 2 ? r.q.z : r.q.w;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // elements 8 CH + 2p, + 1: nibbles 2p, 2p + 1 of word CH
      const uint32_t lo = __builtin_amdgcn_ubfe(v, 8 * p, 4), hi = __builtin_amdgcn_ubfe(v, 8 * p + 4, 4);
      o[p] = gw_dq2(lo | (hi << 16), s, c);
    }
  }
};

// Q8_0 split layout (qweight int8 [N, K], fp16 scales [N, K/32])
struct GWQ80S {
  static constexpr int NL = 3;
  struct Raw { u32x4 a, b; uint32_t d; };
  __device__ static void load(const GemmRows& s, uint32_t row, int kt, int h, bool valid, Raw& r) {
    const uint32_t e0 = 64u * (uint32_t)kt + 32u * (uint32_t)h;
    const uint32_t wo = valid ? row * s.rb + e0 : kOOB;
    r.a = bld16(s.w, wo);
    r.b = bld16(s.w, wo + 16u);
    r.d = bld2(s.s, valid ? row * s.sb + 2u * (e0 / 32u) : kOOB);
  }
  template <int CH>
  __device__ static void decode(const Raw& r, int, uint32_t (&o)[4], int) {
    const float d = h2f(r.d), s = d * 16777216.f, c = -128.f * d;
    const uint32_t w[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t q = w[2 * CH + k] ^ 0x80808080u;
      o[2 * k] = gw_dq2(__builtin_amdgcn_perm(0u, q, 0x0c010c00u), s, c);
      o[2 * k + 1] = gw_dq2(__builtin_amdgcn_perm(0u, q, 0x0c030c02u), s, c);
    }
  }
};

// Q5_0 split layout (qweight u8 [N, K/2]: byte j holds elements 2j (low nibble) and
// 2j + 1 (high); qhigh u8 [N, K/2]: their fifth bits in bits 0 and 4; fp16 scales)
struct GWQ50S {
  static constexpr int NL = 3;
  static constexpr int MAXMI = 2;                // (a 256x256 tile spills)
  struct Raw { u32x4 q, hq; uint32_t d; };
  __device__ static void load(const GemmRows& s, uint32_t row, int kt, int h, bool valid, Raw& r) {
    const uint32_t e0 = 64u * (uint32_t)kt + 32u * (uint32_t)h;
    const uint32_t wo = valid ? row * s.rb + e0 / 2u : kOOB;
    r.q = bld16(s.w, wo);
    r.hq = bld16(s.aux, wo);
    r.d = bld2(s.s, valid ? row * s.sb + 2u * (e0 / 32u) : kOOB);
  }
  template <int CH>
  __device__ static void decode(const Raw& r, int, uint32_t (&o)[4], int) {
    const float d = h2f(r.d), s = d * 16777216.f, c = -16.f * d;
    const uint32_t q = CH == 0 ? r.q.x : CH == 1 ? r.q.y : CH == 2 ? r.q.z : r.q.w;
    const uint32_t hq = CH == 0 ? r.hq.x : CH == 1 ? r.hq.y : CH == 2 ? r.hq.z : r.hq.w;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // elements 8 CH + 2p, + 1 from byte p of word CH: (lo nibble | bit 0 << 4, hi nibble | bit 4)
      const uint32_t lo = __builtin_amdgcn_ubfe(q, 8 * p, 4) | (__builtin_amdgcn_ubfe(hq, 8 * p, 1) << 4);
      const uint32_t hi = __builtin_amdgcn_ubfe(q, 8 * p + 4, 4) | (__builtin_amdgcn_ubfe(hq, 8 * p + 4, 1) << 4);
      o[p] = gw_dq2(lo | (hi << 16), s, c);
    }
  }
};

// Q6_K wire blocks (210 B per 256): step kt is quarter j = kt % 4 of super-block kt / 4,
// elements 128 hh + 32 s + l with hh = j / 2 and s = 2 (j % 2) + t; thread h takes
// t = h: low bits = 32 ql bytes at 64 hh + 32 h (nibble j % 2), high bits = 32 qh
// bytes at 128 + 32 hh (bits 2 s), scales bytes 192 + 8 hh + 2 s (+1 for l >= 16), d
// at 208.  The runs are loaded from the 4-byte boundary below them and realigned.
struct GWQ6K {
  static constexpr int NL = 8;
  static constexpr int MAXMI = 2;                // (a 256x256 tile spills)
  struct Raw { uint32_t ql[9], qh[9], sc, d, sh; };
  __device__ static void load(const GemmRows& s, uint32_t row, int kt, int h, bool valid, Raw& r) {
    const uint32_t j = (uint32_t)kt & 3u, hh = j >> 1;
    const uint32_t bo = row * s.rb + 210u * ((uint32_t)kt >> 2), sh = bo & 2u;
    const uint32_t base = valid ? bo - sh : kOOB;
    const uint32_t qo = base + 64u * hh + 32u * (uint32_t)h, ho = base + 128u + 32u * hh;
    const u32x4 a0 = bld16(s.w, qo), a1 = bld16(s.w, qo + 16u);
    const u32x4 b0 = bld16(s.w, ho), b1 = bld16(s.w, ho + 16u);
    r.ql[0] = a0.x; r.ql[1] = a0.y; r.ql[2] = a0.z; r.ql[3] = a0.w;
    r.ql[4] = a1.x; r.ql[5] = a1.y; r.ql[6] = a1.z; r.ql[7] = a1.w;
    r.ql[8] = bld4(s.w, qo + 32u);
    r.qh[0] = b0.x; r.qh[1] = b0.y; r.qh[2] = b0.z; r.qh[3] = b0.w;
    r.qh[4] = b1.x; r.qh[5] = b1.y; r.qh[6] = b1.z; r.qh[7] = b1.w;
    r.qh[8] = bld4(s.w, ho + 32u);
    const uint32_t so = valid ? bo + 192u + 8u * hh + 4u * (j & 1u) + 2u * (uint32_t)h : kOOB;
    r.sc = bld2(s.w, so);
    r.d = bld2(s.w, valid ? bo + 208u : kOOB);
    r.sh = 8u * sh;
  }
  __device__ static uint32_t al(uint32_t hi, uint32_t lo, uint32_t shb) {
    return (uint32_t)(((uint64_t)hi << 32 | lo) >> shb);
  }
  template <int CH>
  __device__ static void decode(const Raw& r, int h, uint32_t (&o)[4], int kt) {
    const uint32_t j = (uint32_t)kt & 3u, s6 = 2u * (j & 1u) + (uint32_t)h;
    const uint32_t nsh = 4u * (j & 1u), qsh = 2u * s6;
    // l < 16 (chunks 0, 1): the first of the two scales
    const float sc = h2f(r.d) * (float)(int8_t)((r.sc >> (CH < 2 ? 0 : 8)) & 0xFFu);
    const float sm = sc * 16777216.f, c = -32.f * sc;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      constexpr int i0 = 2 * CH;
      const int i = i0 + k;
      const uint32_t v = al(r.ql[i + 1], r.ql[i], r.sh), u = al(r.qh[i + 1], r.qh[i], r.sh);
      const uint32_t q4 = ((v >> nsh) & 0x0F0F0F0Fu) | (((u >> qsh) & 0x03030303u) << 4);
      o[2 * k] = gw_dq2(__builtin_amdgcn_perm(0u, q4, 0x0c010c00u), sm, c);
      o[2 * k + 1] = gw_dq2(__builtin_amdgcn_perm(0u, q4, 0x0c030c02u), sm, c);
    }
  }
};

// largest tile row factor (64 MI rows) a provider's registers allow: 4 unless stated
template <class W, class = void>
struct GwMaxMi : std::integral_constant<int, 4> {};
template <class W>
struct GwMaxMi<W, std::void_t<decltype(W::MAXMI)>> : std::integral_constant<int, W::MAXMI> {};

// a provider's 128x256-tile rate relative to its 256x256 tile: 0.79 unless stated
template <class W, class = void>
struct GwR128 { static constexpr double value = 0.79; };
template <class W>
struct GwR128<W, std::void_t<decltype(W::R128)>> { static constexpr double value = W::R128; };

// provider load shim (MLX needs the group size)
template <class W>
__device__ __forceinline__ void gw_load(const GemmRows& s, uint32_t row, int kt, int h, bool valid,
                                        typename W::Raw& r, int gs) {
  if constexpr (std::is_same<W, GWMLX>::value) W::load(s, row, kt, h, valid, r, gs);
  else W::load(s, row, kt, h, valid, r);
}

template <class W, int MI, typename YT>
__global__ __launch_bounds__(512) void k_gemm_w(GemmArgs ga, const f16* x, int M, YT* y, int N, int K, int gs) {
  const GemmRows g(ga);
  constexpr int QBM = 64 * MI, QBN = 256, NI = 2;
  __shared__ __attribute__((aligned(1024))) uint8_t xs0[QBM * 128], xs1[QBM * 128], xs2[QBM * 128];
  __shared__ __attribute__((aligned(1024))) uint8_t ws0[QBN * 128], ws1[QBN * 128];
  uint8_t* const XS[3] = {xs0, xs1, xs2};
  uint8_t* const WS[2] = {ws0, ws1};
  const int KT = K / 64;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wm = wave >> 2, wn = wave & 3;
  const int m0 = (int)blockIdx.y * QBM, n0 = (int)blockIdx.x * QBN;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), ALLOY_RSRC_DW3);

  uint32_t xoff[MI];
#pragma unroll
  for (int i = 0; i < MI; ++i) {
    const int r = 8 * (MI * wave + i) + (lane >> 3), c = (lane & 7) ^ lds_swz(r);
    xoff[i] = ((uint32_t)(m0 + r) * (uint32_t)K + 8u * (uint32_t)c) * 2u;
  }
  auto xcopy = [&](int kt, uint8_t* st) {
    const uint32_t so = 128u * (uint32_t)kt;
#pragma unroll
    for (int i = 0; i < MI; ++i) lds_copy16(xr, st + 1024 * (MI * wave + i), kt < KT ? xoff[i] : kOOB, so);
  };

  const int br = tid % QBN, h = tid / QBN;                      // h uniform per wave
  const uint32_t row = (uint32_t)(n0 + br);
  const bool row_in = n0 + br < N;
  const int swb = lds_swz(br);
  typename W::Raw raw[3];
  auto rload = [&](int kt, typename W::Raw& slot) { gw_load<W>(g, row, kt, h, row_in && kt < KT, slot, gs); };
  auto deq = [&](const typename W::Raw& slot, auto chc, int kt, uint8_t* st) {
    constexpr int CH = decltype(chc)::value;
    uint32_t o[4];
    W::template decode<CH>(slot, h, o, kt);
    *(u32x4*)(st + br * 128 + (((4 * h + CH) ^ swb) << 4)) = u32x4{o[0], o[1], o[2], o[3]};
  };

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

  // step kt (J = kt % 6): MFMAs on x stage kt%3 and weight stage kt%2; x(kt+2) copied
  // first; step kt+1's weights (ring slot (kt+1)%3) decoded into weight stage
  // (kt+1)%2 between the MFMA substeps; step kt+4's bytes loaded into that slot last
  auto step = [&](auto Jc, int kt) {
    constexpr int J = decltype(Jc)::value;
    constexpr int R1 = (J + 1) % 3;
    const uint8_t* xc = XS[J % 3];
    const uint8_t* wc = WS[J & 1];
    xcopy(kt + 2, XS[(J + 2) % 3]);
    frag(xc, wc, 0, 0);
    xs_static_for<0, 4>([&](auto ksc) {
      constexpr int ks = decltype(ksc)::value, cs = ks & 1;
      if constexpr (ks < 3) frag(xc, wc, ks + 1, cs ^ 1);
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int jn = 0; jn < NI; ++jn)
          acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cs][i], bf[cs][jn], acc[i][jn], 0, 0, 0);
      deq(raw[R1], ksc, kt + 1, WS[(J + 1) & 1]);      // chunk ks of step kt+1's weights
    });
    __builtin_amdgcn_sched_barrier(0);
    rload(kt + 4, raw[R1]);
    // a full wait at the end of every even step: x(k) (issued at step k-2) is needed at
    // step k, the weights of step p (issued at the end of step p-4) at step p-1, so a
    // full wait lies between every load and its first use; odd steps order the LDS
    // stages only
    if constexpr ((J & 1) == 0) step_barrier<0>();
    else step_barrier_lds();
  };

  // prologue: steps 0..2 loaded (slots 0..2), x of steps 0 and 1, step 0 decoded into
  // weight stage 0, step 3 into slot 0
#pragma unroll
  for (int p = 0; p < 3; ++p) rload(p, raw[p]);
  xcopy(0, xs0);
  xcopy(1, xs1);
  xs_static_for<0, 4>([&](auto chc) { deq(raw[0], chc, 0, ws0); });
  __builtin_amdgcn_sched_barrier(0);
  rload(3, raw[0]);
  step_barrier<0>();                                     // x(0) and x(1) landed
  int kt = 0;
  for (; kt + 6 <= KT; kt += 6) {
    step(std::integral_constant<int, 0>(), kt + 0);
    step(std::integral_constant<int, 1>(), kt + 1);
    step(std::integral_constant<int, 2>(), kt + 2);
    step(std::integral_constant<int, 3>(), kt + 3);
    step(std::integral_constant<int, 4>(), kt + 4);
    step(std::integral_constant<int, 5>(), kt + 5);
  }
  // 0..5 more steps
  if (kt < KT) step(std::integral_constant<int, 0>(), kt + 0);
  if (kt + 1 < KT) step(std::integral_constant<int, 1>(), kt + 1);
  if (kt + 2 < KT) step(std::integral_constant<int, 2>(), kt + 2);
  if (kt + 3 < KT) step(std::integral_constant<int, 3>(), kt + 3);
  if (kt + 4 < KT) step(std::integral_constant<int, 4>(), kt + 4);

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
  // slices in groups of four: the group's loads are all requested before the first
  // add (one memory latency per group, not per slice); summed in slice order
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int z0 = 0; z0 < S; z0 += 4) {
    f32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {        // past the last slice: the last slice again (unused)
      const int z = z0 + k < S ? z0 + k : S - 1;
      v[k] = *(const f32x4*)(ws + (int64_t)z * mn + i);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (z0 + k < S) acc = z0 + k == 0 ? v[k] : acc + v[k];
  }
  if constexpr (sizeof(YT) == 4) {
    *(f32x4*)((float*)y + i) = acc;
  } else {
    const float a0 = acc[0], a1 = acc[1], a2 = acc[2], a3 = acc[3];   // elements copied out first
    *(f16x4*)((f16*)y + i) = f16x4{(f16)a0, (f16)a1, (f16)a2, (f16)a3};
  }
}

hipError_t launch_splitk_sum(const float* ws, int S, int64_t mn, void* y, bool y_f32, hipStream_t st) {
  if (mn % 4 || ((uintptr_t)ws & 15) || ((uintptr_t)y & (y_f32 ? 15 : 7))) return hipErrorNotSupported;
  const int64_t blocks = (mn / 4 + 255) / 256;
  if (y_f32) hipLaunchKernelGGL(k_splitk_sum<float>, dim3((unsigned)blocks), dim3(256), 0, st, ws, S, mn, (float*)y);
  else hipLaunchKernelGGL(k_splitk_sum<f16>, dim3((unsigned)blocks), dim3(256), 0, st, ws, S, mn, (f16*)y);
  return hipGetLastError();
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

// other formats on the swizzled kernel: tile 256x256, 128x256 or 64x256 by the same
// last-round fill score as the Q4_K plan (no K split); hipErrorNotSupported when the
// shape does not fit it (K not a multiple of 64 / 256 for Q6_K, fp32 activations,
// buffers of 2 GiB or more, MLX group size not a multiple of 32)
template <class W>
static hipError_t launch_gemm_w(int fmt, const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32, int64_t M,
                                int64_t N, const Opts& o, hipStream_t st) {
  const int64_t K = a.K;
  if (x_f32 || K % (fmt == F_Q6_K ? 256 : 64) || (fmt == F_MLX && (a.gs < 32 || a.gs % 32)))
    return hipErrorNotSupported;
  const uint32_t sb = fmt == F_MLX ? (uint32_t)(2 * (K / a.gs)) : (fmt == F_Q8_0S || fmt == F_Q5_0S) ? (uint32_t)(2 * (K / 32)) : 0u;
  if ((uint64_t)M * (uint64_t)K * 2u >= (1ull << 31) || (uint64_t)N * (uint64_t)a.rb >= (1ull << 31) ||
      (uint64_t)N * sb >= (1ull << 31) || (uint64_t)M * (uint64_t)N * 4u >= (1ull << 31))
    return hipErrorNotSupported;
  GemmArgs g{a.w, a.aux, a.s, a.b, (uint32_t)N * (uint32_t)a.rb, (uint32_t)N * sb, (uint32_t)a.rb, sb};
  // forced tile (variants 4, 5, 7 = 256x256, 128x256, 64x256), else the fill score
  int mi = o.variant == 4 ? 4 : o.variant == 5 ? 2 : o.variant == 7 ? 1 : 0;
  if (!mi) {
    const int cus = cu_count();
    const int bm[3] = {256, 128, 64}, mis[3] = {4, 2, 1};
    // measured at M = 2048 on the config 3 / 4 shapes (MLX: the 128x256 tile is slower)
    const double rate[3] = {1000e12, GwR128<W>::value * 1000e12, 0.59 * 1000e12};
    double best = 1e30;
    for (int k = GwMaxMi<W>::value >= 4 ? 0 : 1; k < 3; ++k) {
      const int64_t wg = ((M + bm[k] - 1) / bm[k]) * ((N + 255) / 256), rounds = (wg + cus - 1) / cus;
      const double t = 1.0 / (rate[k] * (double)wg / (double)(rounds * cus));
      if (t < best) { best = t; mi = mis[k]; }
    }
  }
  auto go = [&](auto mic) {
    constexpr int MI = decltype(mic)::value;
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)((M + 64 * MI - 1) / (64 * MI)));
    if (y_f32)
      hipLaunchKernelGGL((k_gemm_w<W, MI, float>), grid, dim3(512), 0, st, g, (const f16*)x, (int)M, (float*)y, (int)N,
                         (int)K, a.gs);
    else
      hipLaunchKernelGGL((k_gemm_w<W, MI, f16>), grid, dim3(512), 0, st, g, (const f16*)x, (int)M, (f16*)y, (int)N,
                         (int)K, a.gs);
    return hipGetLastError();
  };
  if (mi > GwMaxMi<W>::value) mi = GwMaxMi<W>::value;
  if constexpr (GwMaxMi<W>::value >= 4) {
    if (mi == 4) return go(std::integral_constant<int, 4>());
  }
  if (mi == 2) return go(std::integral_constant<int, 2>());
  return go(std::integral_constant<int, 1>());
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
  // the other formats: the swizzled kernel unless the 128x128 kernel is forced (variant
  // 1) or the shape does not fit it
  if (fmt != F_Q4_K && M > 64 && o.variant != 1) {
    hipError_t e = hipErrorNotSupported;
    switch (fmt) {
      case F_Q8_0: e = launch_gemm_w<GWQ80>(fmt, a, x, x_f32, y, y_f32, M, N, o, st); break;
      case F_Q5_0: e = launch_gemm_w<GWQ50>(fmt, a, x, x_f32, y, y_f32, M, N, o, st); break;
      case F_Q6_K: e = launch_gemm_w<GWQ6K>(fmt, a, x, x_f32, y, y_f32, M, N, o, st); break;
      case F_MLX: e = launch_gemm_w<GWMLX>(fmt, a, x, x_f32, y, y_f32, M, N, o, st); break;
      case F_Q8_0S: e = launch_gemm_w<GWQ80S>(fmt, a, x, x_f32, y, y_f32, M, N, o, st); break;
      case F_Q5_0S: e = launch_gemm_w<GWQ50S>(fmt, a, x, x_f32, y, y_f32, M, N, o, st); break;
      default: break;
    }
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();
  }
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
