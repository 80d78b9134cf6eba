// Dense quantized matmul kernels for gfx950: dequant probe, quantized embedding,
// M=1 GEMV (v_dot2), M<=16 GEMV on MFMA and the gated pair (the prefill GEMM is in
// gemm.hip).  All launched on the caller's
// HIP stream; no allocation, no global mutable state.
#include <map>
#include <mutex>
#include <tuple>
#include <type_traits>

#include "gemv.h"
#include "launch.h"
#include "xs.h"

namespace alloy {

// ------------------------------------------------------------------ dequant probe
// One thread per (row, 32-element group).  out is [nrows, K] f32 (exact) or f16 (RN).
template <class F>
__global__ __launch_bounds__(256) void k_dequant(QArgs a, void* out, int out_f16, int64_t row0,
                                                 int64_t nrows) {
  const int64_t groups = a.K >> 5;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= nrows * groups) return;
  const int64_t r = t / groups;
  const int k0 = (int)(t - r * groups) * 32;
  float w[32];
  F::dec32(a, row0 + r, k0, w);
  const int64_t o = r * a.K + k0;
  if (out_f16) {
    f16* p = (f16*)out + o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      f16x8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (f16)w[8 * j + e];
      *(f16x8*)(p + 8 * j) = v;
    }
  } else {
    float* p = (float*)out + o;
#pragma unroll
    for (int j = 0; j < 8; ++j) *(f32x4*)(p + 4 * j) = f32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
  }
}

// ------------------------------------------------------------------ quantized embedding
// One thread per (id, 32-element group): out[i, :] = exact fp32 decode of row ids[i];
// ids outside [0, N) give zero rows (no weight bytes are read for them).
template <class F>
__global__ __launch_bounds__(256) void k_embed(QArgs a, const void* ids, int ids64, int64_t n_ids, int64_t N,
                                               float* out) {
  const int64_t groups = a.K >> 5;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n_ids * groups) return;
  const int64_t i = t / groups;
  const int k0 = (int)(t - i * groups) * 32;
  const int64_t id = ids64 ? ((const int64_t*)ids)[i] : (int64_t)((const int32_t*)ids)[i];
  float w[32];
  if (id >= 0 && id < N) {
    F::dec32(a, id, k0, w);
  } else {
#pragma unroll
    for (int e = 0; e < 32; ++e) w[e] = 0.f;
  }
  float* p = out + i * a.K + k0;
#pragma unroll
  for (int j = 0; j < 8; ++j) *(f32x4*)(p + 4 * j) = f32x4{w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
}

template <class F>
struct EmbedRun {
  static hipError_t run(const QArgs& a, const void* ids, bool ids64, int64_t n_ids, int64_t N, float* out,
                        hipStream_t st) {
    const int64_t work = n_ids * (a.K >> 5);
    if (work == 0) return hipSuccess;
    hipLaunchKernelGGL(k_embed<F>, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, st, a, ids, (int)ids64, n_ids,
                       N, out);
    return hipGetLastError();
  }
};

// ------------------------------------------------------------------ M=1 GEMV (v_dot2)
// Each thread owns UPT decode units of the row (the same units for every row it
// visits) and keeps their x values in registers: fp16 pairs in the format's XPERM
// order plus fp32 sums per 16 elements.  L threads cover one row (L >= units per
// row / UPT), so a 256-thread workgroup works on 256/L rows at a time and walks
// its rows with a grid stride; the next row's weight bytes are loaded while the
// current row is computed.  Row sums are reduced in a fixed order (shuffles inside
// a wave, then LDS across waves).  grid.y = activation row.
template <class F, int UPT, int D, typename XT>
__global__ __launch_bounds__(256) void k_gemv_dot2(QArgs a, const XT* x, void* y, int y_f32,
                                                   int64_t N, int C16) {
  __shared__ float red[2][16];
  const int L = 16 * C16;
  const int R = blockDim.x / L;
  const int K = a.K, U = K / F::UE;
  const int t = threadIdx.x, slot = t / L, li = t - slot * L;
  const int64_t m = blockIdx.y;
  bool own[UPT];
  int uu[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    own[j] = li + L * j < U;
    uu[j] = own[j] ? li + L * j : U - 1;     // clamped unit: always a valid address
  }
  const int64_t stride = (int64_t)gridDim.x * R;
  const int64_t nb0 = (int64_t)blockIdx.x * R;
  auto clamp_row = [&](int64_t n) { return n < N ? n : N - 1; };
  typename F::Raw ring[D][UPT];
#pragma unroll
  for (int d = 0; d < D; ++d)
#pragma unroll
    for (int j = 0; j < UPT; ++j) ring[d][j] = F::load(a, clamp_row(nb0 + d * stride + slot), uu[j]);
  uint32_t xr[UPT][F::UE / 2];
  float xg[UPT][F::UE / 16];
  const XT* xm = x + m * K;
#pragma unroll
  for (int j = 0; j < UPT; ++j) load_x_unit<F, XT>(xm, uu[j], xr[j], xg[j]);

  int par = 0;
  // Sum of slot d's row (all lanes of the row end with the sum), then refill slot d.
  auto step = [&](int d, int64_t n) {
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      const float v = F::dot(ring[d][j], uu[j], xr[j], xg[j]);
      acc += own[j] ? v : 0.f;
    }
#pragma unroll
    for (int j = 0; j < UPT; ++j) ring[d][j] = F::load(a, clamp_row(n + D * stride), uu[j]);
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (C16 > 1) {
      if ((li & 15) == 0) red[par][slot * C16 + (li >> 4)] = acc;
      __syncthreads();
      acc = 0.f;
      for (int g = 0; g < C16; ++g) acc += red[par][slot * C16 + g];
      par ^= 1;
    }
    return acc;
  };
  int64_t base = nb0;
  // full blocks: every row of every slot is in range, every lane stores its row sum
  for (; base + (int64_t)(D - 1) * stride + R <= N; base += D * stride) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int64_t n = base + d * stride + slot;
      const float v = step(d, n);
      store_y(y, y_f32, m * N + n, v);
    }
  }
  // tail
  for (; base < N; base += D * stride) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int64_t nbd = base + d * stride;     // uniform
      if (nbd >= N) break;
      const int64_t n = nbd + slot;
      const float v = step(d, n);
      if (li == 0 && n < N) store_y(y, y_f32, m * N + n, v);
    }
  }
}

// ------------------------------------------------------------------ M=1 GEMV, wave rows
// L = 16, 32 or 64 lanes share a row inside one wave (64/L rows per wave, 256/L per
// workgroup); each lane owns UPT decode units of the row, the same for every row
// it visits, with their x in registers.  Weights stream through a ring of D rows
// per lane by raw buffer loads: offsets are 32-bit, and rows past N read as zero
// (no clamps, no faults), so every refill is unconditional.  A row's partial sums
// reduce across its L lanes with DPP (quad_perm, row mirrors, row_bcast 15/31) —
// no LDS, no barrier — and the row's last lane stores it.
template <class F, int UPT, int D, typename XT, typename YT, int NB>
__device__ __forceinline__ void gemv_w_body(const WaveBatchT<NB>& bt, uint32_t sb, const XT* x, int lshift) {
  // this workgroup's matrix: the batch entry whose block range holds blockIdx.x
  // (uniform; single-matrix launches are batches of one, NB = 1)
  int mi = 0;
#pragma unroll
  for (int i = 1; i < NB; ++i) mi = (i < bt.n && (int)blockIdx.x >= bt.b0[i]) ? i : mi;
  const QArgs a = bt.a[mi];
  YT* const y = (YT*)bt.y[mi];
  const int64_t ldy = bt.ldy[mi];
  const int N = bt.N[mi];
  const int bx = (int)blockIdx.x - bt.b0[mi], gx = bt.b0[mi + 1] - bt.b0[mi];
  const int L = 1 << lshift;
  const int t = threadIdx.x, li = t & (L - 1), slot = t >> lshift;
  const int R = blockDim.x >> lshift;
  const int K = a.K, U = K / F::UE;
  const int64_t m = blockIdx.y;
  const uint32_t rb = (uint32_t)a.rb;
  const Src src(a, (uint32_t)N * rb, (uint32_t)N * sb);
  // output row m as a buffer: every lane stores, lanes other than a group's last one
  // (and rows >= N) aim past the end, so the hardware drops them — no branch
  constexpr uint32_t esz = sizeof(YT);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(y + m * ldy), (short)0, (int)((uint32_t)N * esz), ALLOY_RSRC_DW3);
  bool own[UPT];
  int uu[UPT];
  uint32_t wo[UPT], so[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = li + L * j;
    own[j] = u < U;
    uu[j] = own[j] ? u : U - 1;            // x of a valid unit; result dropped
    // a unit past the row's end loads from past the buffer's end: zeros, no traffic
    wo[j] = own[j] ? F::woff(a, uu[j]) : 0x80000000u;
    so[j] = own[j] ? F::soff(a, uu[j]) : 0x80000000u;
  }
  const int stride = gx * R;
  const int n0 = bx * R + slot;
  uint32_t rw = (uint32_t)n0 * rb, rs = (uint32_t)n0 * sb;   // row offsets of ring slot 0
  const uint32_t dw = (uint32_t)stride * rb, ds = (uint32_t)stride * sb;
  // Activation row m reaches the lanes through LDS: one coalesced copy per workgroup
  // (global -> registers, issued before the weight ring so the wait for it leaves the
  // ring in flight, -> LDS), then each lane reads the x of its units.  Loading x per
  // lane from global memory instead re-reads the same few KiB for every row slot of
  // every workgroup, which costs L1/L2 cycles comparable to the weights themselves.
  static_assert(std::is_same<XT, f16>::value, "wave-row GEMV takes fp16 activations");
  constexpr int XV = 512 * F::UE / 4096;          // 16-byte chunks per thread at the largest K
  __shared__ __attribute__((aligned(16))) f16 xl[256 * F::UE];
  const uint32_t xbytes = 2u * (uint32_t)K;
  const __amdgpu_buffer_rsrc_t xrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(x + m * K), (short)0, (int)xbytes, ALLOY_RSRC_DW3);
  u32x4 xv[XV];
#pragma unroll
  for (int i = 0; i < XV; ++i)
    if (4096u * i < xbytes) xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (uint32_t)t * 16u + 4096u * i, 0, 0);
  typename F::Raw ring[D][UPT];
#pragma unroll
  for (int d = 0; d < D; ++d)
#pragma unroll
    for (int j = 0; j < UPT; ++j) ring[d][j] = F::load_b(src, rw + d * dw + wo[j], rs + d * ds + so[j], uu[j]);
#pragma unroll
  for (int i = 0; i < XV; ++i)
    if (4096u * i < xbytes) *(u32x4*)((uint8_t*)xl + t * 16 + 4096 * i) = xv[i];
  lds_barrier_asm();
  uint32_t xr[UPT][F::UE / 2];
  float xg[UPT][F::UE / 16];
#pragma unroll
  for (int j = 0; j < UPT; ++j) load_x_unit<F, f16>(xl, uu[j], xr[j], xg[j]);
  const bool odd = li & 1;
  if constexpr (HasPairDot<F>::value) {
#pragma unroll
    for (int j = 0; j < UPT; ++j) F::pair_x_sums(xg[j], odd);
  }

  for (int base = bx * R; base < N; base += D * stride) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int nb = base + d * stride;      // uniform across the workgroup
      // leave the kernel, not just the unrolled steps: a jump to the loop latch would
      // merge a state with only some slots refilled into the loop head and force a
      // full vmcnt wait there
      if (nb >= N) return;
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < UPT; ++j) {
        if constexpr (HasShare<F>::value) F::share(ring[d][j]);
        if constexpr (HasPairDot<F>::value) {
          acc += F::dot_pair(ring[d][j], uu[j], xr[j], xg[j], odd);   // (units past the row add 0)
        } else {
          const float v = F::dot(ring[d][j], uu[j], xr[j], xg[j]);
          acc += own[j] ? v : 0.f;
        }
      }
      const uint32_t nw = rw + (d + D) * dw, ns = rs + (d + D) * ds;
#pragma unroll
      for (int j = 0; j < UPT; ++j) ring[d][j] = F::load_b(src, nw + wo[j], ns + so[j], uu[j]);
      acc = dpp_sum_rows(acc, lshift);
      const uint32_t yo = li == L - 1 ? (uint32_t)(nb + slot) * esz : 0x80000000u;
      if constexpr (sizeof(YT) == 4) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), yr, yo, 0, 0);
      else __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (f16)acc), yr, yo, 0, 0);
    }
    rw += D * dw;
    rs += D * ds;
  }
}

template <class F, int UPT, int D, typename XT, typename YT, int NB>
__global__ __launch_bounds__(256) void k_gemv_w(WaveBatchT<NB> bt, uint32_t sb, const XT* x, int lshift) {
  gemv_w_body<F, UPT, D, XT, YT, NB>(bt, sb, x, lshift);
}

// One matrix with its arguments as scalars, which the dispatch can preload into
// SGPRs (a structure argument is always read from memory first, a round trip on the
// critical path of a short launch); the most used first.
template <class F, int UPT, int D, typename XT, typename YT>
__global__ __launch_bounds__(256) void k_gemv_w1(const uint8_t* w, int64_t rb, int K, const XT* x, void* y, int N,
                                                 int lshift, uint32_t sb, int64_t ldy, const uint16_t* sc,
                                                 const uint16_t* bi, const uint8_t* aux, int gs) {
  WaveBatchT<1> bt;
  bt.n = 1;
  bt.b0[0] = 0;
  bt.b0[1] = (int)gridDim.x;
  bt.a[0] = QArgs{w, aux, sc, bi, rb, gs, K};
  bt.y[0] = y;
  bt.ldy[0] = ldy;
  bt.N[0] = N;
  gemv_w_body<F, UPT, D, XT, YT, 1>(bt, sb, x, lshift);
}

// ------------------------------------------------------------------ M<=16 GEMV on MFMA
// v_mfma_f32_16x16x32_f16 with A = 16 weight rows (dequantised to fp16 in registers),
// B = x^T (up to 16 activation rows).  A K-chunk of 128 elements is split over the
// four 16-lane quarters (32 elements each, pieces of 8 per MFMA); the four waves of a
// workgroup take chunks round-robin and are reduced through LDS in a fixed order.
template <class F, int RG, typename XT>
__global__ __launch_bounds__(256) void k_gemv_mfma(QArgs a, const XT* x, int M, void* y,
                                                   int y_f32, int64_t N) {
  __shared__ float red[3][RG][64][4];
  const int K = a.K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int i = lane & 15, kq = lane >> 4;
  const int64_t nb = (int64_t)blockIdx.x * 16 * RG;
  const int mcol0 = blockIdx.y * 16;                     // x rows handled: mcol0 .. +16
  const int mrow = mcol0 + i;
  f32x4 acc[RG];
#pragma unroll
  for (int r = 0; r < RG; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 128 * wave; k0 < K; k0 += 512) {
    const int kk = k0 + 32 * kq;
    const bool kin = kk < K;
    f16x8 bfr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (kin && mrow < M) bfr[j] = ld_x8<XT>(x + (int64_t)mrow * K + kk + 8 * j);
      else bfr[j] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
#pragma unroll
    for (int r = 0; r < RG; ++r) {
      const int64_t n = nb + 16 * r + i;
      f16x8 afr[4];
      if (kin && n < N) dec32_f16<F>(a, n, kk, afr);
      else {
#pragma unroll
        for (int j = 0; j < 4; ++j) afr[j] = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(afr[j], bfr[j], acc[r], 0, 0, 0);
    }
  }
  // fixed-order cross-wave reduction: wave 0 adds waves 1, 2, 3 in order
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < RG; ++r)
#pragma unroll
      for (int t = 0; t < 4; ++t) red[wave - 1][r][lane][t] = acc[r][t];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int r = 0; r < RG; ++r) {
#pragma unroll
      for (int w = 0; w < 3; ++w)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[r][t] += red[w][r][lane][t];
      // D[row 4kq + t][col i]  ->  y[x row mcol0 + i][weight row nb + 16r + 4kq + t]
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int64_t n = nb + 16 * r + 4 * kq + t;
        if (mrow < M && n < N) store_y(y, y_f32, (int64_t)mrow * N + n, acc[r][t]);
      }
    }
  }
}

// ------------------------------------------------------------------ M <= 16 GEMV, Q4_K, 4x4x4 MFMA
// A wave owns 64 weight rows (one per lane) and a fixed range of SPW super-blocks of
// K; the W waves of a workgroup cover all of K for the same 64 rows and are reduced
// through LDS in a fixed order.  v_mfma_f32_4x4x4_16b_f16 with CBSZ = 4 broadcasts
// block ABID's A operand to all 16 blocks, so lane 4b + t holds x[token t] at k-slice
// b of each 64-element pair chunk and one register pair feeds 16 MFMAs; each lane's
// B operand is 4 elements of its own row.  D: lane 4b + j holds row 4b + j's sums
// for four tokens.  Quants enter B as the exact fp16 integers 1024 + q (low nibble)
// or 1024 + 16q (high nibble) by one v_bfi_b32 each, in element order (0, 2, 1, 3)
// per word (x is permuted alike).  Per sub-block, with s = d*sc, c = -dmin*m:
//   y += s'*D + (c - 1024 s')*X,   s' = s (low) or s/16 (high),
// X = the sub-block's x sum per token, computed once per wave (ones operand) into LDS.
constexpr int M4_MAXW = 16;

template <int ABID>
__device__ __forceinline__ f32x4 mfma4_bcast(f16x4 a, f16x4 b, f32x4 c) {   // A from block ABID
  return __builtin_amdgcn_mfma_f32_4x4x4f16(a, b, c, 4, ABID, 0);
}
template <int I, int N, class Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    static_for<I + 1, N>(f);
  }
}

// up to 16 waves, or 8 when the x operands need more than 64 VGPRs
template <int TG, int SPW>
constexpr int m4_max_threads() { return TG * SPW >= 4 ? 512 : 1024; }

template <int TG, int T1, int SPW, typename YT>
__global__ __launch_bounds__((m4_max_threads<TG, SPW>())) void k_gemv_q4k_m4(QArgs a, const f16* x, int M, YT* y, int N) {
  // TG token groups of 4 (M <= 4 TG); T1: tokens used in each group (1 when M == 1)
  __shared__ __attribute__((aligned(16))) float Xs[M4_MAXW][SPW * 8][TG][4];
  __shared__ __attribute__((aligned(16))) float red[M4_MAXW][64][TG * 4];
  const int K = a.K, KSB = K >> 8;
  const int W = (int)(blockDim.x >> 6), wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int blk = lane >> 2, t4 = lane & 3;
  const int sb0 = wave * SPW;                          // first super-block of this wave
  const uint32_t rb = (uint32_t)a.rb;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.w, (short)0, (int)((uint32_t)N * rb), ALLOY_RSRC_DW3);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), ALLOY_RSRC_DW3);

  // raw bytes of one super-block of this lane's row: header + 128 quant bytes
  struct SB { u32x4 hd, q[8]; };
  auto sload = [&](int rg, int s, SB& r) {   // rows past N / super-blocks past K: zero or unused
    const uint32_t bo = (uint32_t)(rg * 64 + lane) * rb + (uint32_t)(sb0 + s) * 144u;
    r.hd = bld16(wr, bo);
#pragma unroll
    for (int c = 0; c < 8; ++c) r.q[c] = bld16(wr, bo + 16u + 16u * c);
  };
  SB pre;                                   // first super-block of the next row group
  sload(blockIdx.x, 0, pre);                // in flight while x is prepared

  // x operands: [group][super-block][pair] -> 4 halves (x at 4 k, order 0,2,1,3)
  f16x4 xa[TG][SPW][4];
#pragma unroll
  for (int g = 0; g < TG; ++g)
#pragma unroll
    for (int s = 0; s < SPW; ++s)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int tok = 4 * g + t4;
        const uint32_t k = (uint32_t)(sb0 + s) * 256u + 64u * p + 4u * blk;
        // rows past M and super-blocks past K read as zero (buffer bounds)
        const uint32_t off = (tok < M && sb0 + s < KSB) ? ((uint32_t)tok * (uint32_t)K + k) * 2u : 0x80000000u;
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(xr, off, 0, 0));
        const uint2 pv = {__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u)};
        xa[g][s][p] = __builtin_bit_cast(f16x4, pv);
      }
  // per-token sums of every sub-block of this wave's range (ones operand), into LDS
  {
    const f16x4 ones = {1, 1, 1, 1};
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int s = 0; s < SPW; ++s)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
          static_for<0, 8>([&](auto ic) {
            constexpr int i = decltype(ic)::value;
            lo = mfma4_bcast<i>(xa[g][s][p], ones, lo);
            hi = mfma4_bcast<8 + i>(xa[g][s][p], ones, hi);
          });
          if (lane == 0) {
            *(f32x4*)Xs[wave][8 * s + 2 * p][g] = lo;
            *(f32x4*)Xs[wave][8 * s + 2 * p + 1][g] = hi;
          }
        }
  }
  __syncthreads();

  const uint32_t magic = 0x64006400u;                  // fp16 1024.0 in both halves
  const int ngroups = (N + 63) >> 6;
  for (int rg = blockIdx.x; rg < ngroups; rg += gridDim.x) {
    f32x4 yacc[TG];
#pragma unroll
    for (int g = 0; g < TG; ++g) yacc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
    SB sbuf[2];
    sbuf[0] = pre;
#pragma unroll
    for (int s = 0; s < SPW; ++s) {
      // the next super-block (or the next row group's first) loads during this one
      if (s + 1 < SPW) sload(rg, s + 1, sbuf[(s + 1) & 1]);
      else sload(rg + (int)gridDim.x, 0, pre);
      if (sb0 + s >= KSB) continue;                    // uniform per wave
      const u32x4 hd = sbuf[s & 1].hd;
      const u32x4* q = sbuf[s & 1].q;
      const float d = h2f(hd.x), dmin = h2f(hd.x >> 16);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        uint32_t sc0, mn0, sc1, mn1;
        q4k_scale_min(hd.y, hd.z, hd.w, 2 * p, sc0, mn0);       // constant sub-block
        q4k_scale_min(hd.y, hd.z, hd.w, 2 * p + 1, sc1, mn1);
        const float slo = d * (float)sc0, shi = d * (float)sc1 * 0.0625f;
        const float clo = -(dmin * (float)mn0) - 1024.f * slo, chi = -(dmin * (float)mn1) - 1024.f * shi;
        f32x4 dlo[TG], dhi[TG];
#pragma unroll
        for (int g = 0; g < TG; ++g) dlo[g] = dhi[g] = f32x4{0.f, 0.f, 0.f, 0.f};
        static_for<0, 8>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          const u32x4 qc = q[2 * p + (i >> 2)];
          const uint32_t w = (i & 3) == 0 ? qc.x : (i & 3) == 1 ? qc.y : (i & 3) == 2 ? qc.z : qc.w;
          const uint32_t w8 = w >> 8;
          // plain expressions, not inline asm: the hazard recognizer must see these
          // VGPR writes, which can land in registers an earlier MFMA is still reading
          const f16x4 blo = __builtin_bit_cast(f16x4, uint2{(w & 0x000F000Fu) | magic, (w8 & 0x000F000Fu) | magic});
          const f16x4 bhi = __builtin_bit_cast(f16x4, uint2{(w & 0x00F000F0u) | magic, (w8 & 0x00F000F0u) | magic});
#pragma unroll
          for (int g = 0; g < TG; ++g) {
            dlo[g] = mfma4_bcast<i>(xa[g][s][p], blo, dlo[g]);
            dhi[g] = mfma4_bcast<8 + i>(xa[g][s][p], bhi, dhi[g]);
          }
        });
#pragma unroll
        for (int g = 0; g < TG; ++g) {
          const f32x4 xlo = *(const f32x4*)Xs[wave][8 * s + 2 * p][g];
          const f32x4 xhi = *(const f32x4*)Xs[wave][8 * s + 2 * p + 1][g];
#pragma unroll
          for (int t = 0; t < T1; ++t) {
            const float vlo = dlo[g][t], vhi = dhi[g][t];
            yacc[g][t] += slo * vlo + clo * xlo[t] + shi * vhi + chi * xhi[t];
          }
        }
      }
    }
#pragma unroll
    for (int g = 0; g < TG; ++g) *(f32x4*)&red[wave][lane][4 * g] = yacc[g];
    __syncthreads();
    // fixed-order sum over the waves: thread -> (row, token)
    for (int e = threadIdx.x; e < 64 * TG * 4; e += blockDim.x) {
      const int r = e / (TG * 4), tk = e - r * (TG * 4);
      const int tokg = tk;                             // token index 4g + t
      float v = 0.f;
      for (int ww = 0; ww < W; ++ww) v += red[ww][r][tk];
      const int n = rg * 64 + r;
      if (n < N && tokg < M && ((tokg & 3) < T1)) y[(int64_t)tokg * N + n] = (YT)v;
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------ host launchers

namespace {
std::mutex g_occ_mu;
std::map<std::tuple<int, const void*, int, size_t>, int> g_occ;   // (device, kernel, threads, lds)
std::map<int, int> g_cus;                                           // device -> compute units
}  // namespace

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> g(g_occ_mu);
  auto it = g_cus.find(dev);
  if (it != g_cus.end()) return it->second;
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  g_cus[dev] = v;
  return v;
}

int resident_per_cu(const void* kern, int threads, size_t lds) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  const auto key = std::make_tuple(dev, kern, threads, lds);
  std::lock_guard<std::mutex> g(g_occ_mu);
  auto it = g_occ.find(key);
  if (it != g_occ.end()) return it->second;
  int v = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kern, threads, lds) != hipSuccess || v <= 0) v = 1;
  g_occ[key] = v;
  return v;
}
template <template <class> class Fn, typename... Args>
static hipError_t by_fmt(int fmt, Args&&... args) {
  switch (fmt) {
    case F_Q8_0: return Fn<FQ80>::run(args...);
    case F_Q5_0: return Fn<FQ50>::run(args...);
    case F_Q4_K: return Fn<FQ4K>::run(args...);
    case F_Q6_K: return Fn<FQ6K>::run(args...);
    case F_MLX: return Fn<FMLX>::run(args...);
    case F_Q8_0S: return Fn<FQ80S>::run(args...);
    case F_Q5_0S: return Fn<FQ50S>::run(args...);
    default: return hipErrorInvalidValue;
  }
}

template <class F>
struct DequantRun {
  static hipError_t run(const QArgs& a, void* out, bool out_f16, int64_t row0, int64_t nrows,
                        hipStream_t st) {
    const int64_t work = nrows * (a.K >> 5);
    if (work == 0) return hipSuccess;
    const int64_t blocks = (work + 255) / 256;
    hipLaunchKernelGGL(k_dequant<F>, dim3((unsigned)blocks), dim3(256), 0, st, a, out,
                       (int)out_f16, row0, nrows);
    return hipGetLastError();
  }
};

hipError_t launch_dequant(int fmt, const QArgs& a, void* out, bool out_f16, int64_t row0,
                          int64_t nrows, hipStream_t st) {
  return by_fmt<DequantRun>(fmt, a, out, out_f16, row0, nrows, st);
}

hipError_t launch_embedding(int fmt, const QArgs& a, const void* ids, bool ids64, int64_t n_ids, int64_t N,
                            float* out, hipStream_t st) {
  return by_fmt<EmbedRun>(fmt, a, ids, ids64, n_ids, N, out, st);
}

static int pow2_floor(int v) {
  int p = 1;
  while (p * 2 <= v) p *= 2;
  return p;
}

template <class F>
struct GemvDot2Run {
  template <int UPT, typename XT>
  static hipError_t go(const QArgs& a, const void* x, void* y, bool y_f32, int64_t M, int64_t N,
                       int C16, int grid_cap, int depth, hipStream_t st) {
    const int R = 16 / C16;
    int64_t grid = (N + R - 1) / R;
    const int64_t cap = grid_cap > 0 ? grid_cap : 1024;
    if (grid > cap) grid = cap;
    const dim3 g((unsigned)grid, (unsigned)M), b(16 * C16 * R);
    if (depth == 2)
      hipLaunchKernelGGL((k_gemv_dot2<F, UPT, 2, XT>), g, b, 0, st, a, (const XT*)x, y, (int)y_f32, N, C16);
    else if (depth == 4)
      hipLaunchKernelGGL((k_gemv_dot2<F, UPT, 4, XT>), g, b, 0, st, a, (const XT*)x, y, (int)y_f32, N, C16);
    else
      hipLaunchKernelGGL((k_gemv_dot2<F, UPT, 3, XT>), g, b, 0, st, a, (const XT*)x, y, (int)y_f32, N, C16);
    return hipGetLastError();
  }
  static hipError_t run(const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32, int64_t M,
                        int64_t N, const Opts& o, hipStream_t st) {
    const int U = a.K / F::UE;
    // threads per row: one unit each when U <= 256, else two; in groups of 16
    int upt = U > 256 ? 2 : 1;
    int C16 = ((U + upt - 1) / upt + 15) / 16;
    if (o.lanes_per_row >= 16) {                     // explicit override (tuning / tests)
      const int c = o.lanes_per_row / 16;
      if (c * 16 * 2 >= U) { C16 = c > 16 ? 16 : c; upt = C16 * 16 >= U ? 1 : 2; }
    }
    if (upt == 2) return x_f32 ? go<2, float>(a, x, y, y_f32, M, N, C16, o.grid_cap, o.depth, st)
                               : go<2, f16>(a, x, y, y_f32, M, N, C16, o.grid_cap, o.depth, st);
    return x_f32 ? go<1, float>(a, x, y, y_f32, M, N, C16, o.grid_cap, o.depth, st)
                 : go<1, f16>(a, x, y, y_f32, M, N, C16, o.grid_cap, o.depth, st);
  }
};

// Wave-row GEMV launcher.  Returns hipErrorNotSupported when the shape needs more
// than 4 units per lane at 64 lanes per row (then the LDS-combining kernel runs).
template <class F>
struct GemvWaveRun {
  template <int UPT, int D, typename YT>
  static hipError_t go(const WaveBatch& b, uint32_t sb, const void* x, int64_t M, int lshift, int grid_cap,
                       hipStream_t st) {
    if (b.n == 1) return go_n<UPT, D, YT, 1>(b, sb, x, M, lshift, grid_cap, st);   // small arguments
    return go_n<UPT, D, YT, kMaxBatch>(b, sb, x, M, lshift, grid_cap, st);
  }
  template <int UPT, int D, typename YT, int NB>
  static hipError_t go_n(const WaveBatch& b, uint32_t sb, const void* x, int64_t M, int lshift, int grid_cap,
                         hipStream_t st) {
    // workgroups per matrix: one per R rows while the total fits the cap, else a
    // share of the cap proportional to the rows (at least one each)
    const int R = 256 >> lshift;
    const int64_t cap = grid_cap > 0 ? grid_cap : 1024;
    int64_t want = 0, rows = 0;
    for (int i = 0; i < b.n; ++i) { want += (b.N[i] + R - 1) / R; rows += b.N[i]; }
    WaveBatchT<NB> bt{};
    bt.n = b.n;
    int acc = 0;
    for (int i = 0; i < b.n; ++i) {
      bt.a[i] = b.a[i];
      bt.y[i] = b.y[i];
      bt.ldy[i] = b.ldy[i];
      bt.N[i] = b.N[i];
      bt.b0[i] = acc;
      int64_t g = (b.N[i] + R - 1) / R;
      if (want > cap) {
        const int64_t share = cap * b.N[i] / (rows > 0 ? rows : 1);
        g = share < 1 ? 1 : share < g ? share : g;
      }
      acc += (int)g;
    }
    bt.b0[b.n] = acc;
    if constexpr (NB == 1) {
      const QArgs& a = bt.a[0];
      hipLaunchKernelGGL((k_gemv_w1<F, UPT, D, f16, YT>), dim3((unsigned)acc, (unsigned)M), dim3(256), 0, st, a.w,
                         a.rb, a.K, (const f16*)x, bt.y[0], bt.N[0], lshift, sb, bt.ldy[0], a.s, a.b, a.aux, a.gs);
    } else {
      hipLaunchKernelGGL((k_gemv_w<F, UPT, D, f16, YT, NB>), dim3((unsigned)acc, (unsigned)M), dim3(256), 0, st,
                         bt, sb, (const f16*)x, lshift);
    }
    return hipGetLastError();
  }
  template <int UPT, typename YT>
  static hipError_t pick_d(int depth, const WaveBatch& b, uint32_t sb, const void* x, int64_t M, int lshift,
                           int cap, hipStream_t st) {
    if (depth == 1) return go<UPT, 1, YT>(b, sb, x, M, lshift, cap, st);
    return go<UPT, 2, YT>(b, sb, x, M, lshift, cap, st);
  }
  template <typename YT>
  static hipError_t pick(int upt, int depth, const WaveBatch& b, uint32_t sb, const void* x, int64_t M,
                         int lshift, int cap, hipStream_t st) {
    switch (upt) {
      case 1: return pick_d<1, YT>(depth, b, sb, x, M, lshift, cap, st);
      case 2: return pick_d<2, YT>(depth, b, sb, x, M, lshift, cap, st);
      case 3: return pick_d<3, YT>(depth, b, sb, x, M, lshift, cap, st);
      default: return pick_d<4, YT>(depth, b, sb, x, M, lshift, cap, st);
    }
  }
  // one matrix: a batch of one
  static hipError_t run(const QArgs& a, uint32_t sb, const void* x, bool x_f32, void* y, int64_t ldy,
                        bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st) {
    WaveBatch b{};
    b.n = 1;
    b.a[0] = a;
    b.y[0] = y;
    b.ldy[0] = ldy;
    b.N[0] = (int)N;
    return run_batch(b, sb, x, x_f32, y_f32, M, o, st);
  }
  // b.n matrices sharing K, the format and x; b.b0 is filled here
  static hipError_t run_batch(const WaveBatch& b, uint32_t sb, const void* x, bool x_f32, bool y_f32, int64_t M,
                              const Opts& o, hipStream_t st) {
    if (x_f32) return hipErrorNotSupported;         // fp32 activations: ring kernel
    const QArgs& a = b.a[0];
    int64_t N = 0;
    for (int i = 0; i < b.n; ++i) N += b.N[i];
    const int U = a.K / F::UE;
    int lshift;
    if (o.lanes_per_row == 16 || o.lanes_per_row == 32 || o.lanes_per_row == 64)
      lshift = o.lanes_per_row == 16 ? 4 : o.lanes_per_row == 32 ? 5 : 6;
    else {
      lshift = U <= 64 ? 4 : U <= 128 ? 5 : 6;          // at most 4 units per lane
      // short matrices: more lanes per row until there are >= 512 workgroups
      while (lshift < 6 && (N << lshift) < 512 * 256) ++lshift;
    }
    const int L = 1 << lshift;
    const int upt = (U + L - 1) / L;
    if (upt > 4) return hipErrorNotSupported;
    // one row in flight per lane, latency hidden by occupancy: measured at least as
    // fast as a two-row register ring on every decode shape
    const int depth = o.depth == 2 ? 2 : 1;
    // up to three workgroups per CU (two at four units per lane, where the register
    // budget leaves three resident), looping when the rows need more; very tall
    // matrices (lm_head) with eight per CU — measured on the decode shapes
    const int cus = cu_count();
    const int cap = o.grid_cap > 0 ? o.grid_cap : (N > 32768 ? 8 * cus : upt >= 4 ? 2 * cus : 3 * cus);
    return y_f32 ? pick<float>(upt, depth, b, sb, x, M, lshift, cap, st)
                 : pick<f16>(upt, depth, b, sb, x, M, lshift, cap, st);
  }
};

template <class F>
struct GemvWaveBatchRun {
  static hipError_t run(const WaveBatch& b, uint32_t sb, const void* x, bool x_f32, bool y_f32, const Opts& o,
                        hipStream_t st) {
    return GemvWaveRun<F>::run_batch(b, sb, x, x_f32, y_f32, 1, o, st);
  }
};

// bytes per row of the scale / bias buffers the wave kernel views (MLX, split layouts)
static uint32_t scale_row_bytes(int fmt, const QArgs& a) {
  return fmt == F_MLX ? (uint32_t)(2 * (a.K / a.gs)) : (fmt == F_Q8_0S || fmt == F_Q5_0S) ? (uint32_t)(2 * (a.K / 32)) : 0u;
}

hipError_t launch_gemv_batched(int fmt, const WaveBatch& b, const void* x, bool x_f32, bool y_f32, const Opts& o,
                               hipStream_t st) {
  if (b.n < 1 || b.n > kMaxBatch) return hipErrorNotSupported;
  const uint32_t sb = scale_row_bytes(fmt, b.a[0]);
  for (int i = 0; i < b.n; ++i) {               // 32-bit buffer offsets within each matrix
    const int64_t rowb = b.a[i].rb > (int64_t)sb ? b.a[i].rb : (int64_t)sb;
    if ((int64_t)(b.N[i] + 1024) * rowb >= ((int64_t)1 << 31) || b.N[i] <= 0) return hipErrorNotSupported;
  }
  return by_fmt<GemvWaveBatchRun>(fmt, b, sb, x, x_f32, y_f32, o, st);
}

hipError_t launch_gemv_dot2(int fmt, const QArgs& a, const void* x, bool x_f32, void* y,
                            bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st) {
  if (M == 0 || N == 0) return hipSuccess;
  // GGUF blocks that are only 2-byte aligned (Q6_K always; Q5_0 / Q8_0 wire blocks
  // once the matrix is large enough to amortise the staging) go through the
  // LDS-staged kernel, which reads global memory with aligned 16-byte loads only
  const bool unaligned_blocks = fmt == F_Q6_K || ((fmt == F_Q5_0 || fmt == F_Q8_0) && N * a.rb >= ((int64_t)16 << 20));
  if (o.variant == 4 || (o.variant == 0 && unaligned_blocks)) {
    const hipError_t e = launch_gemv_tile(fmt, a, x, x_f32, y, y_f32, M, N, o, st);
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();
  }
  if (o.variant == 0 || o.variant == 3) {
    // scale-row bytes (MLX scales/biases, split-layout scales) for the buffer views
    const uint32_t sb = scale_row_bytes(fmt, a);
    // 32-bit buffer offsets: split the rows into ranges below 2 GiB of weights
    const int64_t wrow = a.rb > 0 ? a.rb : 1;
    const int64_t rows = ((int64_t)1 << 31) / (wrow > (int64_t)sb ? wrow : (int64_t)sb) - 1024;
    hipError_t e = hipSuccess;
    for (int64_t r0 = 0; r0 < N && e == hipSuccess; r0 += rows) {
      const int64_t nr = N - r0 < rows ? N - r0 : rows;
      QArgs ar = a;
      ar.w = a.w + r0 * a.rb;
      if (a.aux) ar.aux = a.aux + r0 * a.rb;
      if (a.s) ar.s = a.s + r0 * (sb / 2);
      if (a.b) ar.b = a.b + r0 * (sb / 2);
      e = by_fmt<GemvWaveRun>(fmt, ar, sb, x, x_f32, (uint8_t*)y + r0 * (y_f32 ? 4 : 2), (int64_t)N, y_f32, M, nr, o, st);
    }
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();
  }
  return by_fmt<GemvDot2Run>(fmt, a, x, x_f32, y, y_f32, M, N, o, st);
}

// ------------------------------------------------------------------ M <= 16 GEMV, x-stationary 16x16x32
// Each wave owns a fixed K range and keeps the activations of that range (16 token
// rows, zero past M) as MFMA A operands in registers for the whole kernel; the
// workgroup's W waves cover K for the same weight rows and are reduced through LDS
// in a fixed order.  B = 16 weight rows x one 32-element sub-block, quants as exact
// fp16 integers (1024 + q, high nibbles 1024 + 16q); D (lane: row l%16, tokens
// 4(l/16)+t) is fresh per sub-block and folded in fp32 as y += s*D + c*X with the
// sub-block's scale s, offset c (minus 1024 s) and X = sum of x over the sub-block
// per token (computed once per wave into LDS with a ones operand).  Q4_K x is
// permuted (0,2,1,3) per 4 elements to match the unpack order.
template <int NS, int TT, int XS_RT, typename YT>
__global__ __launch_bounds__(1024) void k_gemv_xs_q4k(QArgs a, const f16* x, int M, YT* y, int N) {
  // NS: sub-blocks (of 32) per wave, a multiple of 8 (whole super-blocks); TT: tokens
  // folded per lane (1 when M == 1, else 4); XS_RT: 16-row tiles per LDS reduction,
  // whose weight bytes are all requested before any of them is used
  __shared__ __attribute__((aligned(16))) float Xs[16][NS][16];
  __shared__ __attribute__((aligned(16))) float red[16][XS_RT][64][4];
  const int K = a.K;
  const int W = (int)(blockDim.x >> 6), wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n16 = lane & 15, kq = lane >> 4;
  const int k0 = wave * NS * 32;                 // first element of this wave's range
  const int nsb = (K - k0) / 32 < NS ? (K - k0) / 32 : NS;   // sub-blocks present (multiple of 8)
  const uint32_t rb = (uint32_t)a.rb;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)a.w, (short)0, (int)((uint32_t)N * rb), ALLOY_RSRC_DW3);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)((uint32_t)M * (uint32_t)K * 2u), ALLOY_RSRC_DW3);
  // A operands: token n16, elements 32s + 8kq + (0,2,1,3, 4,6,5,7)
  f16x8 xa[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t off = (n16 < M && s < nsb) ? ((uint32_t)n16 * (uint32_t)K + (uint32_t)(k0 + 32 * s + 8 * kq)) * 2u
                                              : 0x80000000u;
    const u32x4 v = bld16(xr, off);
    const u32x4 pv = {__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                      __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
    xa[s] = __builtin_bit_cast(f16x8, pv);
  }
  {
    const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const f32x4 X = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s], ones, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      if (n16 == 0) *(f32x4*)&Xs[wave][s][4 * kq] = X;   // tokens 4kq .. 4kq+3
    }
  }
  __syncthreads();

  const uint32_t magic = 0x64006400u;
  const int ntiles = (N + 15) >> 4;
  for (int t0 = blockIdx.x * XS_RT; t0 < ntiles; t0 += gridDim.x * XS_RT) {
    // all weight bytes of the tiles first (one memory round trip), then the math
    u32x4 hd[XS_RT][NS / 8];
    uint2 qw[XS_RT][NS / 8][4];
#pragma unroll
    for (int r = 0; r < XS_RT; ++r) {
      const int n = (t0 + r) * 16 + n16;           // rows past N read zero
#pragma unroll
      for (int sb = 0; sb < NS / 8; ++sb) {        // super-blocks past K: unused
        const uint32_t bo = (uint32_t)n * rb + (uint32_t)((k0 >> 8) + sb) * 144u;
        hd[r][sb] = bld16(wr, bo);
#pragma unroll
        for (int p = 0; p < 4; ++p)
          qw[r][sb][p] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, bo + 16u + 32u * p + 8u * kq, 0, 0));
      }
    }
#pragma unroll
    for (int r = 0; r < XS_RT; ++r) {
      f32x4 yacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sb = 0; sb < NS / 8; ++sb) {        // super-blocks of this wave's range
        if (sb >= nsb / 8) break;                  // uniform; keeps xa[] statically indexed
        const u32x4 h = hd[r][sb];
        const float d = h2f(h.x), dmin = h2f(h.x >> 16);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          uint32_t sc0, mn0, sc1, mn1;
          q4k_scale_min(h.y, h.z, h.w, 2 * p, sc0, mn0);
          q4k_scale_min(h.y, h.z, h.w, 2 * p + 1, sc1, mn1);
          const float slo = d * (float)sc0, shi = d * (float)sc1 * 0.0625f;
          const float clo = -(dmin * (float)mn0) - 1024.f * slo, chi = -(dmin * (float)mn1) - 1024.f * shi;
          const uint32_t w0 = qw[r][sb][p].x, w1 = qw[r][sb][p].y, w08 = w0 >> 8, w18 = w1 >> 8;
          const u32x4 blo = {(w0 & 0x000F000Fu) | magic, (w08 & 0x000F000Fu) | magic,
                             (w1 & 0x000F000Fu) | magic, (w18 & 0x000F000Fu) | magic};
          const u32x4 bhi = {(w0 & 0x00F000F0u) | magic, (w08 & 0x00F000F0u) | magic,
                             (w1 & 0x00F000F0u) | magic, (w18 & 0x00F000F0u) | magic};
          const int s = 8 * sb + 2 * p;
          const f32x4 dlo = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s], __builtin_bit_cast(f16x8, blo), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          const f32x4 dhi = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[s + 1], __builtin_bit_cast(f16x8, bhi), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          const f32x4 xl = *(const f32x4*)&Xs[wave][s][4 * kq], xh = *(const f32x4*)&Xs[wave][s + 1][4 * kq];
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            const float vl = dlo[t], vh = dhi[t];
            yacc[t] += slo * vl + clo * xl[t] + shi * vh + chi * xh[t];
          }
        }
      }
      *(f32x4*)red[wave][r][lane] = yacc;
    }
    __syncthreads();
    // fixed-order sum over the waves; thread -> (tile r, lane l, token slot t)
    for (int e = threadIdx.x; e < XS_RT * 64 * 4; e += blockDim.x) {
      const int r = e >> 8, l = (e >> 2) & 63, t = e & 3;
      const int tok = 4 * (l >> 4) + t, n = (t0 + r) * 16 + (l & 15);
      float v = 0.f;
      for (int ww = 0; ww < W; ++ww) v += red[ww][r][l][t];
      if (n < N && tok < M && (TT == 4 || t == 0)) y[(int64_t)tok * N + n] = (YT)v;
    }
    __syncthreads();
  }
}

static hipError_t launch_gemv_xs_q4k(const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32,
                                     int64_t M, int64_t N, const Opts& o, hipStream_t st) {
  if (x_f32 || M > 16 || a.K % 256 || (uint64_t)N * (uint64_t)a.rb >= (1ull << 31) ||
      (uint64_t)M * (uint64_t)a.K * 2u >= (1ull << 31))
    return hipErrorNotSupported;
  const int KS = a.K / 32;                        // sub-blocks of K
  int ns = 8;
  while ((KS + ns - 1) / ns > 16) ns *= 2;        // at most 16 waves
  if (ns > 16) return hipErrorNotSupported;       // x of a longer K range would not fit
  const int W = (KS + ns - 1) / ns;
  const int64_t tiles = (N + 15) / 16;
  // one 16-row tile per reduction while that still leaves <= 1024 workgroups
  const int rt = (tiles <= 1024 || ns == 16) ? 1 : 4;   // (16 sub-blocks leave no registers)
  const int64_t groups = (tiles + rt - 1) / rt;
  const int64_t cap = o.grid_cap > 0 ? o.grid_cap : 1024;
  const dim3 grid((unsigned)(groups < cap ? groups : cap)), block((unsigned)(64 * W));
  auto go = [&](auto nsc, auto ttc) -> hipError_t {
    constexpr int NS = decltype(nsc)::value, TT = decltype(ttc)::value;
    auto launch = [&](auto rtc) {
      constexpr int RT = decltype(rtc)::value;
      if (y_f32)
        hipLaunchKernelGGL((k_gemv_xs_q4k<NS, TT, RT, float>), grid, block, 0, st, a, (const f16*)x, (int)M, (float*)y, (int)N);
      else
        hipLaunchKernelGGL((k_gemv_xs_q4k<NS, TT, RT, f16>), grid, block, 0, st, a, (const f16*)x, (int)M, (f16*)y, (int)N);
    };
    if constexpr (NS == 8) {
      if (rt == 4) {
        launch(std::integral_constant<int, 4>());
        return hipGetLastError();
      }
    }
    launch(std::integral_constant<int, 1>());
    return hipGetLastError();
  };
  using T1 = std::integral_constant<int, 1>;
  using T4 = std::integral_constant<int, 4>;
  auto by_ns = [&](auto ttc) -> hipError_t {
    if (ns == 8) return go(std::integral_constant<int, 8>(), ttc);
    return go(std::integral_constant<int, 16>(), ttc);
  };
  return M == 1 ? by_ns(T1()) : by_ns(T4());
}

// Q4_K M <= 16 GEMV on 4x4x4 MFMA; hipErrorNotSupported when the shape does not fit.
static hipError_t launch_gemv_q4k_m4(const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32,
                                     int64_t M, int64_t N, const Opts& o, hipStream_t st) {
  if (x_f32 || M > 16 || a.K % 256 || (uint64_t)N * (uint64_t)a.rb >= (1ull << 31) ||
      (uint64_t)M * (uint64_t)a.K * 2u >= (1ull << 31))
    return hipErrorNotSupported;
  const int KSB = a.K / 256;
  const int TGn = M == 1 ? 1 : M <= 4 ? 1 : M <= 8 ? 2 : 4;
  int spw = 1, W = KSB;
  while (W > (TGn * spw >= 4 ? 8 : 16) && spw <= 4) { ++spw; W = (KSB + spw - 1) / spw; }
  if (spw > 4) return hipErrorNotSupported;
  if (TGn == 4 && spw > 2) {
    // 16 tokens over a long K would not fit the registers: two passes of 8 tokens
    const hipError_t e = launch_gemv_q4k_m4(a, x, x_f32, y, y_f32, 8, N, o, st);
    if (e != hipSuccess) return e;
    return launch_gemv_q4k_m4(a, (const f16*)x + 8 * (int64_t)a.K, x_f32,
                              (uint8_t*)y + 8 * N * (y_f32 ? 4 : 2), y_f32, M - 8, N, o, st);
  }
  const int64_t ngroups = (N + 63) / 64;
  const int64_t cap = o.grid_cap > 0 ? o.grid_cap : 1024;
  const dim3 grid((unsigned)(ngroups < cap ? ngroups : cap)), block((unsigned)(64 * W));
  auto go = [&](auto tg, auto t1, auto sp) -> hipError_t {
    constexpr int TG = decltype(tg)::value, T1 = decltype(t1)::value, SP = decltype(sp)::value;
    if (y_f32)
      hipLaunchKernelGGL((k_gemv_q4k_m4<TG, T1, SP, float>), grid, block, 0, st, a, (const f16*)x, (int)M, (float*)y, (int)N);
    else
      hipLaunchKernelGGL((k_gemv_q4k_m4<TG, T1, SP, f16>), grid, block, 0, st, a, (const f16*)x, (int)M, (f16*)y, (int)N);
    return hipGetLastError();
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using I4 = std::integral_constant<int, 4>;
  auto by_spw = [&](auto tg, auto t1) -> hipError_t {
    switch (spw) {
      case 1: return go(tg, t1, I1());
      case 2: return go(tg, t1, I2());
      case 3: return go(tg, t1, I3());
      default: return go(tg, t1, I4());
    }
  };
  if (M == 1) return by_spw(I1(), I1());
  if (M <= 4) return by_spw(I1(), I4());
  if (M <= 8) return by_spw(I2(), I4());
  return by_spw(I4(), I4());
}

template <class F>
struct GemvMfmaRun {
  template <int RG, typename XT>
  static hipError_t go(const QArgs& a, const void* x, int M, void* y, bool y_f32, int64_t N,
                       hipStream_t st) {
    const int64_t grid = (N + 16 * RG - 1) / (16 * RG);
    const int gy = (M + 15) / 16;
    hipLaunchKernelGGL((k_gemv_mfma<F, RG, XT>), dim3((unsigned)grid, (unsigned)gy), dim3(256), 0, st,
                       a, (const XT*)x, M, y, (int)y_f32, N);
    return hipGetLastError();
  }
  static hipError_t run(const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32, int64_t M,
                        int64_t N, const Opts& o, hipStream_t st) {
    const int rg = o.row_groups == 2 ? 2 : 1;
    if (x_f32) return rg == 2 ? go<2, float>(a, x, (int)M, y, y_f32, N, st) : go<1, float>(a, x, (int)M, y, y_f32, N, st);
    return rg == 2 ? go<2, f16>(a, x, (int)M, y, y_f32, N, st) : go<1, f16>(a, x, (int)M, y, y_f32, N, st);
  }
};

// M <= 16 on the generic x-stationary kernel (Q4_K, Q6_K, MLX with a power-of-two
// group size; GGUF wire Q5_0 / Q8_0 with dequantised weights only); hipErrorNotSupported
// when the format or shape does not fit it.
static hipError_t launch_xs_job(int fmt, XsJob j, const Opts& o, hipStream_t st, bool dq);

// splits > 1 (with ws holding splits M N fp32): K cut into that many ranges of whole
// 256-element units, one grid row of workgroups each writing its fp32 partial slice,
// then the slices summed in order into y (deterministic)
static hipError_t launch_gemv_xs(int fmt, const QArgs& a, const void* x, bool x_f32, void* y, bool y_f32,
                                 int64_t M, int64_t N, const Opts& o, hipStream_t st, bool dq = false,
                                 int splits = 1, float* ws = nullptr) {
  if (x_f32 || M > 16 || N >= (1ll << 31) || (uint64_t)M * (uint64_t)a.K * 2u >= (1ull << 31))
    return hipErrorNotSupported;
  XsJob j{};
  j.a = a;
  j.x = (const f16*)x;
  j.xbytes = (uint32_t)(M * a.K * 2);
  j.xld = a.K;
  j.M = (int)M;
  j.N = (int)N;
  j.y = y;
  j.y_f32 = y_f32;
  const int KU = a.K / 256;
  if (splits > 1 && ws && a.K % 256 == 0 && KU >= 2) {
    const int ku = (KU + splits - 1) / splits;
    const int S = (KU + ku - 1) / ku;
    if (S > 1) {
      j.ku_split = ku;
      j.y = ws;
      j.y_f32 = 1;
      const hipError_t e = launch_xs_job(fmt, j, o, st, dq);
      if (e != hipSuccess) return e;
      return launch_splitk_sum(ws, S, M * N, y, y_f32, st);
    }
  }
  return launch_xs_job(fmt, j, o, st, dq);
}

static hipError_t launch_xs_job(int fmt, XsJob j, const Opts& o, hipStream_t st, bool dq) {
  const QArgs& a = j.a;
  const int64_t M = j.M, N = j.N;
  const int64_t cap = o.grid_cap > 0 ? o.grid_cap : 1024;
  if (dq) {
    // measured on the config 2 / 3 shapes: wide matrices loop one workgroup per CU
    // over their tiles (next tiles' weights in flight); Q4_K at M > 8 on mid-size N
    // takes two tiles per reduction
    const int64_t dcap = o.grid_cap > 0 ? o.grid_cap : N >= 12288 ? cu_count() : 1024;
    const int rt = o.row_groups ? o.row_groups : fmt == F_Q4_K && M > 8 && N > 4096 && N < 12288 ? 2 : 1;
    if (fmt == F_Q4_K) return launch_xs<XsDQ<XsQ4K>, 0>(j, 0, dcap, rt, st);
    if (fmt == F_Q6_K) return launch_xs<XsDQ<XsQ6KW>, 0>(j, 0, dcap, rt, st);
    if (fmt == F_Q5_0) return launch_xs<XsDQ<XsQ50>, 0>(j, 0, dcap, rt, st);
    if (fmt == F_Q8_0) return launch_xs<XsDQ<XsQ80>, 0>(j, 0, dcap, rt, st);
    if (fmt == F_Q8_0S) {
      j.sb = (uint32_t)(a.K / 16);               // fp16 scales per row
      return launch_xs<XsDQ<XsQ80S>, 0>(j, 0, dcap, rt, st);
    }
    if (fmt == F_Q5_0S) {
      j.sb = (uint32_t)(a.K / 16);
      return launch_xs<XsDQ<XsQ50S>, 0>(j, 0, dcap, rt, st);
    }
  } else {
    if (fmt == F_Q4_K) return launch_xs<XsQ4K, 0>(j, 0, cap, o.row_groups, st);
    if (fmt == F_Q6_K) return launch_xs<XsQ6K, 0>(j, 0, cap, o.row_groups, st);
  }
  if (fmt != F_MLX || a.gs < 32 || (a.gs & (a.gs - 1))) return hipErrorNotSupported;
  j.sb = (uint32_t)(a.K / a.gs * 2);
  if (dq) {
    switch (a.gs) {
      case 32: return launch_xs<XsMLXD<0>, 0>(j, 0, cap, o.row_groups, st);
      case 64: return launch_xs<XsMLXD<1>, 0>(j, 0, cap, o.row_groups, st);
      case 128: return launch_xs<XsMLXD<2>, 0>(j, 0, cap, o.row_groups, st);
      default: return a.gs == 256 ? launch_xs<XsMLXD<3>, 0>(j, 0, cap, o.row_groups, st) : hipErrorNotSupported;
    }
  }
  switch (a.gs) {
    case 32: return launch_xs<XsMLX<0>, 0>(j, 0, cap, o.row_groups, st);
    case 64: return launch_xs<XsMLX<1>, 0>(j, 0, cap, o.row_groups, st);
    case 128: return launch_xs<XsMLX<2>, 0>(j, 0, cap, o.row_groups, st);
    default: return a.gs == 256 ? launch_xs<XsMLX<3>, 0>(j, 0, cap, o.row_groups, st) : hipErrorNotSupported;
  }
}

// ------------------------------------------------------------------ gated pair
bool glu_fused_supported(int fmt, int64_t M, int64_t N, int64_t K, bool x_f32, int gs) {
  if (x_f32 || M < 1 || M > 16 || K % 256 || K > 4096 || N >= (1ll << 31)) return false;
  // Fused only where it wins (us per pair, fused against two products + combine).
  // Q4_K loses wherever the products take the v_dot2 GEMVs (M = 1: K 3072 N 8192
  // 15.8 / 12.3, K 2048 N 768 7.1 / 6.3; M = 2, N 768: 7.3 / 6.8) and wins against the
  // MFMA GEMVs (K 4096 N 4096 M = 2: 12.3 / 16.2; K 3072 N 8192 M = 16: 20.0 / 21.1).
  // MLX wins at M = 1 (12.6 / 13.0, 6.4 / 7.3) and M >= 2 (K 3072 N 8192 M = 4: 16.5 /
  // 20.3).  Past N = 8192 both lose (K 4096 N 14336 M = 4: Q4_K 45.2 / 36.1, MLX 43.2 /
  // 36.3).
  if (N > 8192) return false;
  if (fmt == F_Q4_K) return M >= 4 || (M >= 2 && M * N > 6144);
  return fmt == F_MLX && gs >= 32 && gs <= 256 && !(gs & (gs - 1));
}

hipError_t launch_glu_fused(int fmt, int act, const QArgs& g, const QArgs& u, const void* x, bool x_f32,
                            void* y, bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st) {
  if (!glu_fused_supported(fmt, M, N, g.K, x_f32, g.gs)) return hipErrorNotSupported;
  XsJob j{};
  j.a = g;
  j.a2 = u;
  j.act = act;
  j.x = x;
  j.xbytes = (uint32_t)(M * g.K * 2);
  j.xld = g.K;
  j.M = (int)M;
  j.N = (int)N;
  j.y = y;
  j.y_f32 = y_f32;
  const int64_t cap = o.grid_cap > 0 ? o.grid_cap : 0;
  if (fmt == F_Q4_K) return launch_xs<XsQ4K, 3>(j, 0, cap, 0, st);
  j.sb = (uint32_t)(g.K / g.gs * 2);
  switch (g.gs) {
    case 32: return launch_xs<XsMLX<0>, 3>(j, 0, cap, 0, st);
    case 64: return launch_xs<XsMLX<1>, 3>(j, 0, cap, 0, st);
    case 128: return launch_xs<XsMLX<2>, 3>(j, 0, cap, 0, st);
    default: return launch_xs<XsMLX<3>, 3>(j, 0, cap, 0, st);
  }
}

template <typename YT>
__global__ __launch_bounds__(256) void k_glu_combine(const float* g, const float* u, YT* y, int64_t n, int act) {
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    y[i] = (YT)xs_f32_product(xs_act(act, g[i]), u[i]);   // fp32 product, then the conversion
}

hipError_t launch_glu_combine(int act, const float* g, const float* u, void* y, bool y_f32, int64_t n,
                              hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  const dim3 grid((unsigned)(blocks < 4096 ? blocks : 4096));
  if (y_f32) hipLaunchKernelGGL(k_glu_combine<float>, grid, dim3(256), 0, st, g, u, (float*)y, n, act);
  else hipLaunchKernelGGL(k_glu_combine<f16>, grid, dim3(256), 0, st, g, u, (f16*)y, n, act);
  return hipGetLastError();
}

// Default kernel choice for 2 <= M <= 16 (measured on the config 1 / 2 / 3 shapes):
//   Q4_K  tall (N >= 32768) and 3 <= M <= 6: 4x4x4 broadcast kernel; K <= 8192: the
//         x-stationary kernel with fp16-dequantised weights (8); else the Q4_K
//         x-stationary kernel
//   Q6_K, Q5_0, Q8_0 (wire blocks), split Q8_0 / Q5_0  x-stationary with fp16-dequantised
//         weights (K over 4096: in passes over K)
//   MLX   generic x-stationary (exact products); N >= 12288: the dequantising
//         provider with 16-byte loads, one workgroup per CU looping over the tiles
//   other formats (and shapes the above do not take): 16x16x32 kernel
static int mfma_variant(int fmt, int64_t M, int64_t N, int64_t K) {
  if (fmt == F_Q4_K) {
    if (N >= 32768 && M >= 3 && M <= 6) return 5;
    return K <= 8192 ? 8 : 6;
  }
  if (fmt == F_Q6_K || fmt == F_Q5_0 || fmt == F_Q8_0 || fmt == F_Q8_0S || fmt == F_Q5_0S) return 8;
  if (fmt == F_MLX) return N >= 12288 ? 8 : 7;
  return 1;
}

// K splits of the x-stationary kernels (1: none).  Measured at M = 8 / 16 (graph
// replays): with few 16-row tiles the grid leaves most CUs idle and each workgroup's
// chain grows with K; four splits at <= 64 tiles (Q6_K M = 8 14336x1024 30.0 -> 11.5 us,
// 4096x1024 8.9 -> 7.2 us; Q5_0 / Q8_0 / MLX / Q4_K alike), two at <= 128 (M = 16
// 4096x2048 10.7 -> 9.5 us); at 192 tiles and more splits lose (extra partial traffic
// and the summing launch).  K >= 4096 keeps at least four units per split; Q4_K over
// K = 8192 takes the Q4_K x-stationary kernel, which does not split.
// Q4_K, MLX and the split layouts with few activation rows on few rows run the v_dot2
// wave-row kernel at M <= 16 (launch_gemv_mfma), which takes no workspace (split
// Q5_0 4096 x 1024 M = 4: 4.5 against 7.0 us on its x-stationary provider; 4096 x
// 4096 M = 2: 8.7 against 7.3)
static bool dot2_small_m(int fmt, int64_t M, int64_t N) {
  return (fmt == F_Q4_K || fmt == F_MLX || fmt == F_Q8_0S || fmt == F_Q5_0S) && M <= 8 && M * N <= 6144;
}

static int gemv_splits(int fmt, int64_t M, int64_t N, int64_t K) {
  if (M < 8 || M > 16 || K < 4096 || K % 256 || (fmt == F_Q4_K && K > 8192)) return 1;
  if (dot2_small_m(fmt, M, N)) return 1;
  if (fmt != F_Q4_K && fmt != F_Q6_K && fmt != F_Q5_0 && fmt != F_Q8_0 && fmt != F_Q8_0S && fmt != F_Q5_0S &&
      fmt != F_MLX)
    return 1;
  const int64_t tiles = (N + 15) / 16;
  return tiles <= 64 ? 4 : tiles <= 128 ? 2 : 1;
}

int64_t gemv_workspace_bytes(int fmt, int64_t M, int64_t N, int64_t K) {
  if (M < 2 || M > 16 || N <= 0 || K <= 0) return 0;
  const int S = gemv_splits(fmt, M, N, K);
  return S > 1 ? (int64_t)S * M * N * 4 : 0;
}

hipError_t launch_gemv_mfma(int fmt, const QArgs& a, const void* x, bool x_f32, void* y,
                            bool y_f32, int64_t M, int64_t N, const Opts& o, hipStream_t st,
                            void* ws, int64_t ws_bytes) {
  if (M == 0 || N == 0) return hipSuccess;
  // K splits: forced (opts) or planned, when the workspace holds the partials
  int splits = o.splits > 1 ? o.splits : gemv_splits(fmt, M, N, a.K);
  if (splits > 1 && (!ws || ws_bytes < (int64_t)splits * M * N * 4 || (M * N) % 4 || ((uintptr_t)ws & 15) ||
                     ((uintptr_t)y & (y_f32 ? 15 : 7))))
    splits = 1;
  // Q4_K, MLX and split Q8_0 / Q5_0, few activation rows on few rows (M <= 8, M N <= 6144):
  // the v_dot2 wave-row kernel (16-byte aligned units, each decoded once and dotted
  // with every token) beats the MFMA kernels' fixed cost — Q4_K 3072 x 1024 at
  // M = 2 / 4 / 6: 2.9 / 3.9 / 4.8 us against 4.0 / 5.1 / 5.3 us, 8192 x 1024 M = 4 6.4
  // against 10.5; split Q8_0 4096 x 1024 M = 4 3.9 against 7.0; at M N = 8192 the MFMA
  // kernels win (Q4_K M = 4, 3072 x 2048: 5.2 against 6.2)
  if (o.variant == 0 && dot2_small_m(fmt, M, N)) {
    const hipError_t e = launch_gemv_dot2(fmt, a, x, x_f32, y, y_f32, M, N, o, st);
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();
  }
  // few activation rows on few rows: the LDS-staged v_dot2 kernel (weights read once,
  // decoded once per row and token) beats the MFMA kernels' fixed cost — measured on
  // the BASELINE decode shapes at M = 2, 3, 4, 8 and K = 4096 at M = 2..8 on 512-2048
  // rows (Q6_K 4096 x 1024 M = 4: 5.9 against 7.1 us; M = 6: 7.5 against 7.1)
  const bool tile_small_m = fmt == F_Q6_K || fmt == F_Q5_0 || fmt == F_Q8_0
                                ? M * N <= 3072 || (M <= 4 && M * N <= 4096)
                          : fmt == F_Q4_K && M == 2 && (N <= 1024 || a.K >= 8192);
  const int v = o.variant ? o.variant : tile_small_m ? 9 : mfma_variant(fmt, M, N, a.K);
  hipError_t e = hipErrorNotSupported;
  if (v == 9) e = launch_gemv_tile(fmt, a, x, x_f32, y, y_f32, M, N, o, st);
  else if (v == 7) e = launch_gemv_xs(fmt, a, x, x_f32, y, y_f32, M, N, o, st, false, splits, (float*)ws);
  else if (v == 8) e = launch_gemv_xs(fmt, a, x, x_f32, y, y_f32, M, N, o, st, true, splits, (float*)ws);
  else if (v == 6 && fmt == F_Q4_K) e = launch_gemv_xs_q4k(a, x, x_f32, y, y_f32, M, N, o, st);
  else if (v == 5 && fmt == F_Q4_K) e = launch_gemv_q4k_m4(a, x, x_f32, y, y_f32, M, N, o, st);
  if (e != hipErrorNotSupported) return e;
  (void)hipGetLastError();
  if (fmt == F_Q4_K && o.variant == 0 && v != 6) {     // e.g. K over 8192 for the generic kernel
    e = launch_gemv_xs_q4k(a, x, x_f32, y, y_f32, M, N, o, st);
    if (e != hipErrorNotSupported) return e;
    (void)hipGetLastError();
  }
  return by_fmt<GemvMfmaRun>(fmt, a, x, x_f32, y, y_f32, M, N, o, st);
}

}  // namespace alloy
