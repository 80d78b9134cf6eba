// x-stationary MFMA GEMV for up to 16 activation rows (decode M <= 16 and the
// routed-expert MoE GEMVs), gfx950.
//
// Each wave owns a fixed range of K and keeps the activations of that range (16
// token rows, zero past the row count) as v_mfma_f32_16x16x32_f16 A operands in
// registers for the whole kernel; the workgroup's W waves cover all of K for the same
// 16-row weight tiles and are reduced through LDS in a fixed order.  B = 16 weight
// rows x one 32-element sub-block with the quants as exact fp16 integers (1024 + q,
// or 1024 + 16q for a high nibble), so every product is exact; D (lane: weight row
// l%16, tokens 4(l/16)+t) is fresh per sub-block and folded in fp32 as
//     y += s*D + c*X,
// with the sub-block's scale s, offset c (the format's offset minus 1024 s) and X
// the sub-block's activation sum per token, computed once per wave (ones operand)
// into LDS.  Every weight byte of a group of tiles is requested before any is used.
//
// Units: 256 elements of a row (8 sub-blocks); a wave owns NS/8 units.
#pragma once
#include <atomic>
#include <type_traits>
#include "launch.h"

namespace alloy {

constexpr uint32_t kXsMagic = 0x64006400u;     // fp16 1024.0 in both halves

// ---------------------------------------------------------------- format providers
// load(): the lane's bytes of one unit of its row (kq = lane/16 selects the 8
// elements of every sub-block that the lane feeds to the MFMA); bq<J>(): MFMA J's B
// operand; sc<J>(): its scale and offset; xel(J, kq): the element offset in the unit
// of the lane's 8 activations for MFMA J.  CHAIN: consecutive MFMAs that share one
// scale and offset (their products are summed in the MFMA accumulator and folded
// once).  PERM: the x element order that matches the unpack: 4 -> (0,2,1,3) per 4
// elements, 8 -> (0,4,1,5,2,6,3,7).  rw / rs: byte offsets of the row in the weight
// / scale buffers.

// Q4_K: unit = one 144-byte super-block; the lane reads the 16-byte header and bytes
// 8kq .. 8kq+7 of each 32-byte quant pair (low nibbles: sub-block 2p, high: 2p+1).
struct XsQ4K {
  static constexpr int PERM = 4;
  struct Raw { u32x4 hd; uint2 q[4]; };
  __device__ static int xel(int J, int kq) { return 32 * J + 8 * kq; }
  __device__ static void load(const Src& src, uint32_t rw, uint32_t, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 144u;
    r.hd = bld16(src.w, bo);
#pragma unroll
    for (int p = 0; p < 4; ++p)
      r.q[p] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(src.w, bo + 16u + 32u * p + 8u * kq, 0, 0));
  }
  static constexpr int CHAIN = 1;
  template <int J>
  __device__ static u32x4 bq(const Raw& r) {
    constexpr int p = J >> 1;
    constexpr uint32_t m = (J & 1) ? 0x00F000F0u : 0x000F000Fu;
    const uint32_t w0 = r.q[p].x, w1 = r.q[p].y;
    return u32x4{(w0 & m) | kXsMagic, ((w0 >> 8) & m) | kXsMagic, (w1 & m) | kXsMagic, ((w1 >> 8) & m) | kXsMagic};
  }
  template <int J>
  __device__ static void sc(const Raw& r, float& s, float& c) {
    uint32_t scl, mn;
    q4k_scale_min(r.hd.y, r.hd.z, r.hd.w, J, scl, mn);
    s = h2f(r.hd.x) * (float)scl * ((J & 1) ? 0.0625f : 1.f);
    c = -(h2f(r.hd.x >> 16) * (float)mn) - 1024.f * s;
  }
};

// MLX 4-bit affine, group size 32 << GSH: unit = 128 qweight bytes = 32 words of 8
// elements (element e of a word at bits 4e).  The lane reads LW = 1, 2 or 4
// consecutive words per load (LW = 2^min(GSH, 2)); load l of lane kq covers words
// 4 LW l + LW kq + h (h < LW), and MFMA J = LW l + h takes word slot h of load l, so
// the four lanes of one MFMA read four words of one group (a group is 4 << GSH
// words).  Scales and biases of the unit's groups: a row's groups are contiguous.
template <int GSH>
struct XsMLX {
  static constexpr int PERM = 8;
  static constexpr int LW = GSH >= 2 ? 4 : 1 << GSH;    // words per lane load
  static constexpr int G = GSH >= 3 ? 1 : 8 >> GSH;     // groups per unit
  static constexpr int NW = G >= 2 ? G / 2 : 1;         // scale words per unit
  struct Raw { uint32_t q[8]; uint32_t sc[NW], bi[NW]; };
  // element offset within the unit of lane kq's 8 elements for MFMA J
  __device__ static int xel(int J, int kq) { return 8 * (4 * LW * (J / LW) + LW * kq + J % LW); }
  __device__ static void load(const Src& src, uint32_t rw, uint32_t rs, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 128u + 4u * LW * kq;
#pragma unroll
    for (int l = 0; l < 8 / LW; ++l) {
      if constexpr (LW == 1) {
        r.q[l] = bld4(src.w, bo + 16u * l);
      } else if constexpr (LW == 2) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(src.w, bo + 32u * l, 0, 0));
        r.q[2 * l] = v.x; r.q[2 * l + 1] = v.y;
      } else {
        const u32x4 v = bld16(src.w, bo + 64u * l);
        r.q[4 * l] = v.x; r.q[4 * l + 1] = v.y; r.q[4 * l + 2] = v.z; r.q[4 * l + 3] = v.w;
      }
    }
    if constexpr (G == 8) {
      const uint32_t so = rs + 16u * unit;
      const u32x4 s4 = bld16(src.s, so), b4 = bld16(src.b, so);
      r.sc[0] = s4.x; r.sc[1] = s4.y; r.sc[2] = s4.z; r.sc[3] = s4.w;
      r.bi[0] = b4.x; r.bi[1] = b4.y; r.bi[2] = b4.z; r.bi[3] = b4.w;
    } else if constexpr (G == 4) {
      const uint32_t so = rs + 8u * unit;
      const uint2 s2 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(src.s, so, 0, 0));
      const uint2 b2 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(src.b, so, 0, 0));
      r.sc[0] = s2.x; r.sc[1] = s2.y;
      r.bi[0] = b2.x; r.bi[1] = b2.y;
    } else if constexpr (G == 2) {
      r.sc[0] = bld4(src.s, rs + 4u * unit);
      r.bi[0] = bld4(src.b, rs + 4u * unit);
    } else {
      const uint32_t so = rs + 2u * (((uint32_t)unit << 3) >> GSH);
      r.sc[0] = bld2(src.s, so);
      r.bi[0] = bld2(src.b, so);
    }
  }
  static constexpr int CHAIN = GSH >= 3 ? 8 : 1 << GSH;   // MFMAs per group
  template <int J>
  __device__ static u32x4 bq(const Raw& r) {
    const uint32_t w = r.q[J];
    return u32x4{(w & 0x000F000Fu) | kXsMagic, ((w >> 4) & 0x000F000Fu) | kXsMagic,
                 ((w >> 8) & 0x000F000Fu) | kXsMagic, ((w >> 12) & 0x000F000Fu) | kXsMagic};
  }
  template <int J>
  __device__ static void sc(const Raw& r, float& s, float& c) {
    constexpr int g = GSH >= 3 ? 0 : (4 * LW * (J / LW)) / (4 << GSH);   // group within the unit
    s = h2f(r.sc[g >> 1] >> (16 * (g & 1)));
    c = h2f(r.bi[g >> 1] >> (16 * (g & 1))) - 1024.f * s;
  }
};

// ---------------------------------------------------------------- jobs
// MODE 0: dense y[t, n] = x[t] . W[n] for t < M (x [M, xld] fp16, y fp16 or fp32).
// MODE 1: routed gate/up.  Workgroup row y = column tile (expert e, sorted routes
//         p0 .. p0+cnt); token slot t gathers x[token t of the record]; weight rows
//         e*2N + n (gate) and e*2N + N + n (up); h[p0+t, n] = silu(gate) * up (fp16).
// MODE 2: routed down: x = h[p0+t]; weight rows e*N + n; part[p0+t, n] (fp32).
struct XsJob {
  QArgs a;                 // whole matrix (all experts for MODE 1/2)
  uint32_t sb;             // bytes per row of scales / biases (MLX), else 0
  const f16* x;
  uint32_t xbytes;         // bytes of x readable (bounds of the activation buffer)
  int xld;                 // elements per activation row
  int M;                   // MODE 0: activation rows; MODE 1/2: bound on routes per tile
  int N;                   // output rows (per matrix for MODE 1)
  void* y;                 // MODE 0 output [M, N]
  int y_f32;
  const int32_t* tiles;    // MODE 1/2: column tile records, kTileInts ints each
  const int32_t* ntiles;   // number of valid records
  f16* h;                  // MODE 1 output, MODE 2 input
  float* part;             // MODE 2 output
  int W;                   // waves per workgroup (set by the launcher)
};

template <int I, int N, class Fn>
__device__ __forceinline__ void xs_static_for(Fn&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    xs_static_for<I + 1, N>(f);
  }
}

// NS: sub-blocks per wave (8 or 16); TT: token slots folded per lane (lanes 16 kq
// hold tokens 4 kq .. 4 kq + 3, so at most TT <= 4 active rows need only the first
// TT); RT: 16-row tiles per reduction.  The tile loop is
// software-pipelined over two register sets: the weights of the workgroup's next
// RT tiles are requested before the current ones are used (PIPE), and the first
// tiles' weights are requested before the activations are waited for.  Rows past the
// matrix, tiles past the end and activations past the buffers read as zero (buffer
// bounds, no memory traffic); outputs past the valid rows and tokens are not
// stored.  Dynamic LDS: Xs[W][NS][16] + red[W][RT][64][4 NM] floats.
template <class P, int MODE, int NS, int TT, int RT, bool PIPE, class YT>
__global__ __launch_bounds__(1024) void k_gemv_xs(XsJob j) {
  constexpr int NM = MODE == 1 ? 2 : 1;          // weight matrices per output
  constexpr int UPW = NS / 8;                    // units per wave
  constexpr int CH = P::CHAIN, NSC = NS / CH;    // chains of sub-blocks per wave
  using Raw = typename P::Raw;
  extern __shared__ __attribute__((aligned(16))) float xs_smem[];
  const int K = j.a.K, KU = K >> 8;
  // the wave count comes from the arguments (scalar loads), not from blockDim: that
  // is read with a vector load, and one issued after the weight prefetch makes every
  // later wait drain the prefetch too
  const int W = j.W, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* Xs = xs_smem;                                   // [W][NSC][16]
  float* red = xs_smem + W * NSC * 16;                   // [W][RT][64][4 NM]
  const int n16 = lane & 15, kq = lane >> 4;
  const int u0 = wave * UPW;                             // first unit of this wave
  const int nu = KU - u0 < UPW ? KU - u0 : UPW;          // units present (uniform)

  int cnt = j.M, p0 = 0, tok = 0;
  int64_t row0 = 0;                                      // first weight row of the block
  if constexpr (MODE != 0) {
    // the tile count and the record are read together (records exist for every
    // grid row; those past the count are not used).  The uniform values are moved to
    // scalar registers: a loop that reads a vector register filled by a memory load
    // issued before it makes the compiler drain every outstanding load at its entry,
    // which would also wait for the next tiles' weights.
    const int tile = blockIdx.y;
    const int32_t* rec = j.tiles + kTileInts * tile;
    const int nt = __builtin_amdgcn_readfirstlane(*j.ntiles);
    const int e = __builtin_amdgcn_readfirstlane(rec[0]);
    p0 = __builtin_amdgcn_readfirstlane(rec[1]);
    cnt = __builtin_amdgcn_readfirstlane(rec[2]);
    if constexpr (MODE == 1) tok = rec[4 + n16];
    if (tile >= nt) return;                              // uniform per workgroup
    row0 = (int64_t)e * (NM * j.N);
  }
  QArgs ab = j.a;
  ab.w += row0 * j.a.rb;
  if (ab.s) ab.s += row0 * (j.sb / 2);
  if (ab.b) ab.b += row0 * (j.sb / 2);
  const uint32_t rows = (uint32_t)(NM * j.N);
  const Src src(ab, rows * (uint32_t)j.a.rb, rows * j.sb);
  const uint32_t rb = (uint32_t)j.a.rb;
  const int ntiles16 = (j.N + 15) >> 4;
  const int stride = (int)gridDim.x * RT;

  // request the weights of tiles t .. t+RT-1 (tiles past the end: out of bounds)
  auto load_tiles = [&](Raw (&raw)[RT][NM][UPW], int t) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const bool in = t + r < ntiles16;
      const uint32_t n = (uint32_t)((t + r) * 16 + n16);
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
        const uint32_t row = n + (uint32_t)(mi * j.N);
        const uint32_t rw = in ? row * rb : 0x80000000u, rs = in ? row * j.sb : 0x80000000u;
#pragma unroll
        for (int u = 0; u < UPW; ++u) P::load(src, rw, rs, u0 + u, kq, raw[r][mi][u]);
      }
    }
  };

  // A operands: token slot n16, elements 256 u + xel(s % 8, kq) in PERM order
  f16x8 xa[NS];
  auto load_x = [&]() {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)j.x, (short)0, (int)j.xbytes, ALLOY_RSRC_DW3);
    uint32_t xrow = 0x80000000u;                         // past the buffer: zeros
    if (n16 < cnt) {
      int64_t r = n16;
      if constexpr (MODE == 1) r = tok;
      else if constexpr (MODE == 2) r = p0 + n16;
      xrow = (uint32_t)(r * j.xld) * 2u;
    }
    u32x4 v[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint32_t off = (s >> 3) < nu ? xrow + 2u * (uint32_t)(256 * (u0 + (s >> 3)) + P::xel(s & 7, kq))
                                         : 0x80000000u;
      v[s] = bld16(xr, off);
    }
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      u32x4 pv;
      if constexpr (P::PERM == 4)
        pv = u32x4{__builtin_amdgcn_perm(v[s].y, v[s].x, 0x05040100u), __builtin_amdgcn_perm(v[s].y, v[s].x, 0x07060302u),
                   __builtin_amdgcn_perm(v[s].w, v[s].z, 0x05040100u), __builtin_amdgcn_perm(v[s].w, v[s].z, 0x07060302u)};
      else
        pv = u32x4{__builtin_amdgcn_perm(v[s].z, v[s].x, 0x05040100u), __builtin_amdgcn_perm(v[s].z, v[s].x, 0x07060302u),
                   __builtin_amdgcn_perm(v[s].w, v[s].y, 0x05040100u), __builtin_amdgcn_perm(v[s].w, v[s].y, 0x07060302u)};
      xa[s] = __builtin_bit_cast(f16x8, pv);
    }
  };

  // fold the tiles t .. t+RT-1 of `raw` (TTR token slots per lane), reduce over the
  // waves, store
  auto compute_tiles = [&](const Raw (&raw)[RT][NM][UPW], int t, auto ttc) {
    constexpr int TTR = decltype(ttc)::value;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      f32x4 acc[NM];
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) acc[mi] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < UPW; ++u) {
        if (u >= nu) break;                      // uniform; keeps xa[] statically indexed
        xs_static_for<0, 8 / CH>([&](auto cc) {
          constexpr int C = decltype(cc)::value;
          const f32x4 xsum = *(const f32x4*)&Xs[(wave * NSC + (8 / CH) * u + C) * 16 + 4 * kq];
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) {
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
            xs_static_for<0, CH>([&](auto jc) {
              constexpr int J = C * CH + decltype(jc)::value;
              const u32x4 b = P::template bq<J>(raw[r][mi][u]);
              d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[8 * u + J], __builtin_bit_cast(f16x8, b), d, 0, 0, 0);
            });
            float sc, off;
            P::template sc<C * CH>(raw[r][mi][u], sc, off);
#pragma unroll
            for (int tt = 0; tt < TTR; ++tt) {
              const float dv = d[tt];
              acc[mi][tt] += sc * dv + off * xsum[tt];
            }
          }
        });
      }
#pragma unroll
      for (int mi = 0; mi < NM; ++mi)
        *(f32x4*)&red[((wave * RT + r) * 64 + lane) * (4 * NM) + 4 * mi] = acc[mi];
    }
    __syncthreads();
    // fixed-order sum over the waves; thread -> (tile r, lane l, token slot tt)
    for (int e = threadIdx.x; e < RT * 256; e += 64 * W) {
      const int r = e >> 8, l = (e >> 2) & 63, tt = e & 3;
      const int tk = 4 * (l >> 4) + tt, n = (t + r) * 16 + (l & 15);
      if (n >= j.N || tk >= cnt || tt >= TTR) continue;
      float v0 = 0.f, v1 = 0.f;
      for (int ww = 0; ww < W; ++ww) {
        const float* q = &red[((ww * RT + r) * 64 + l) * (4 * NM)];
        v0 += q[tt];
        if constexpr (NM == 2) v1 += q[4 + tt];
      }
      if constexpr (MODE == 0) {
        ((YT*)j.y)[(int64_t)tk * j.N + n] = (YT)v0;
      } else if constexpr (MODE == 1) {
        j.h[(int64_t)(p0 + tk) * j.N + n] = (f16)(v0 * __builtin_amdgcn_rcpf(1.f + __expf(-v0)) * v1);
      } else {
        j.part[(int64_t)(p0 + tk) * j.N + n] = v0;
      }
    }
    __syncthreads();
  };

  Raw ra[RT][NM][UPW];
  int t = blockIdx.x * RT;
  load_x();                                      // x first: its sums overlap the weight loads
  load_tiles(ra, t);
  {
    // X per chain of sub-blocks: tokens 4kq .. 4kq+3 in lane 16 kq
    const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
#pragma unroll
    for (int c = 0; c < NSC; ++c) {
      f32x4 X = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < CH; ++i) X = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa[c * CH + i], ones, X, 0, 0, 0);
      if (n16 == 0) *(f32x4*)&Xs[(wave * NSC + c) * 16 + 4 * kq] = X;
    }
  }
  __syncthreads();
  auto run = [&](auto ttc) {
    if constexpr (PIPE) {
      Raw rc[RT][NM][UPW];
      for (;;) {
        load_tiles(rc, t + stride);
        compute_tiles(ra, t, ttc);
        t += stride;
        if (t >= ntiles16) break;                // uniform
        load_tiles(ra, t + stride);
        compute_tiles(rc, t, ttc);
        t += stride;
        if (t >= ntiles16) break;
      }
    } else {
      for (;;) {
        compute_tiles(ra, t, ttc);
        t += stride;
        if (t >= ntiles16) break;                // uniform
        load_tiles(ra, t);
      }
    }
  };
  run(std::integral_constant<int, TT>());
}

// Compute units of the current device (cached per device).
inline int xs_cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int v = cached[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
  cached[dev].store(v, std::memory_order_relaxed);
  return v;
}

// Workgroups of `kern` with W waves (and the LDS that W implies) resident per CU
// (cached per kernel and W).
template <class Kern>
int xs_resident_per_cu(Kern kern, int W, size_t lds) {
  static std::atomic<int> cached[17];
  int v = cached[W].load(std::memory_order_relaxed);
  if (v > 0) return v;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, kern, 64 * W, lds) != hipSuccess || v <= 0) v = 1;
  cached[W].store(v, std::memory_order_relaxed);
  return v;
}

// Host launcher.  hipErrorNotSupported when the shape does not fit the kernel
// (K not a multiple of 256 or over 8192, offsets of 2 GiB or more): the caller then
// uses another kernel.  MODE 0: one 16-row tile (rt = 1) or two (rt = 2) per
// workgroup while the tiles fit the resident workgroups, else as many workgroups as
// are resident (or `cap`), each looping over tiles with the next tiles' weights in
// flight.  MODE 1/2: grid.y = `tiles_y` column tiles and grid.x = `cap` groups of
// output tiles per column tile (0: chosen here).
template <class P, int MODE>
hipError_t launch_xs(const XsJob& j, int64_t tiles_y, int64_t cap, int rt, hipStream_t st) {
  constexpr int NM = MODE == 1 ? 2 : 1;
  const int K = j.a.K;
  if (K <= 0 || K % 256 || j.M > 16 || j.N <= 0) return hipErrorNotSupported;
  const uint64_t rows = (uint64_t)NM * (uint64_t)j.N + 16u;
  if (rows * (uint64_t)j.a.rb >= (1ull << 31) || rows * j.sb >= (1ull << 31) || j.xbytes >= (1u << 31))
    return hipErrorNotSupported;
  const int KS = K / 32;
  const int ns = KS <= 8 * 16 ? 8 : KS <= 16 * 16 ? 16 : 0;   // at most 16 waves
  if (!ns || (MODE == 1 && ns == 16)) return hipErrorNotSupported;   // (two matrices: 8 sub-blocks)
  if (MODE != 0 && tiles_y > 65535) return hipErrorNotSupported;
  if (MODE != 0 && tiles_y <= 0) return hipSuccess;
  const int W = (KS + ns - 1) / ns;
  const int64_t tiles = (j.N + 15) / 16;
  // 16 sub-blocks per wave leave registers for one tile in flight only
  rt = (ns == 16 || MODE != 0 || rt < 2) ? 1 : 2;
  const int64_t groups = (tiles + rt - 1) / rt;
  const size_t lds = (size_t)W * (ns / P::CHAIN) * 16 * 4 + (size_t)W * rt * 64 * 4 * NM * 4;
  // token slots per lane: a tile holds at most min(M, 16) rows (routed tiles: one
  // route per token and expert, so at most min(T, 16) with j.M = T)
  const int tt = j.M <= 1 ? 1 : j.M == 2 ? 2 : 4;
  // launch `kern`; pipelined kernels get at most the resident workgroups (or cap)
  auto go = [&](auto kern, bool pipe) -> hipError_t {
    if (lds > 65536) {
      const hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) return e;
    }
    int64_t gx = groups;
    if (pipe) {
      const int64_t c = cap > 0 ? cap : (int64_t)xs_resident_per_cu(kern, W, lds) * xs_cu_count();
      gx = groups < c ? groups : c;
    }
    const dim3 grid((unsigned)gx, MODE == 0 ? 1u : (unsigned)tiles_y), block((unsigned)(64 * W));
    XsJob jw = j;
    jw.W = W;
    hipLaunchKernelGGL(kern, grid, block, lds, st, jw);
    return hipGetLastError();
  };
  // whether the tiles outnumber the resident workgroups of the one-pass kernel
  auto many = [&](auto kern) -> bool {
    const int64_t c = cap > 0 ? cap : (int64_t)xs_resident_per_cu(kern, W, lds) * xs_cu_count();
    return groups > c;
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  if constexpr (MODE == 0) {
    auto pick = [&](auto ttc, auto yt) -> hipError_t {
      constexpr int TT = decltype(ttc)::value;
      using YT = decltype(yt);
      if (ns == 16) return go(k_gemv_xs<P, 0, 16, TT, 1, false, YT>, false);
      if (rt == 2) return go(k_gemv_xs<P, 0, 8, TT, 2, true, YT>, true);
      if (many(k_gemv_xs<P, 0, 8, TT, 1, false, YT>)) return go(k_gemv_xs<P, 0, 8, TT, 1, true, YT>, true);
      return go(k_gemv_xs<P, 0, 8, TT, 1, false, YT>, false);
    };
    if (j.y_f32) return tt == 1 ? pick(I1(), 0.f) : tt == 2 ? pick(I2(), 0.f) : pick(I4(), 0.f);
    return tt == 1 ? pick(I1(), (f16)0) : tt == 2 ? pick(I2(), (f16)0) : pick(I4(), (f16)0);
  } else {
    auto pick = [&](auto ttc) -> hipError_t {
      constexpr int TT = decltype(ttc)::value;
      if constexpr (MODE == 2) {
        if (ns == 16) return go(k_gemv_xs<P, 2, 16, TT, 1, false, float>, false);
      }
      // enough workgroups to fill the chip; beyond that, loop over output tiles (the
      // gathered activations are loaded once per workgroup)
      const int64_t c = cap > 0 ? cap : (2048 + tiles_y - 1) / tiles_y;
      if (groups > c) {
        cap = c;
        return go(k_gemv_xs<P, MODE, 8, TT, 1, true, float>, true);
      }
      return go(k_gemv_xs<P, MODE, 8, TT, 1, false, float>, false);
    };
    return tt == 1 ? pick(I1()) : tt == 2 ? pick(I2()) : pick(I4());
  }
}

}  // namespace alloy
