// Routed-expert MoE over MLX 4-bit and GGUF (Q4_K gate/up, Q6_K down) experts for
// gfx950.
//
// Pipeline (all on the caller's stream, deterministic, no float atomics):
//   1. k_router     per token: top-k logits (ties -> lowest index), softmax over k
//                   (reference: packages/alloy-metal/src/alloy/std/moe.py:31-79)
//   2. k_sort       one workgroup: stable counting sort of the T*k routes by expert
//                   (order within an expert = route order), inverse permutation, and
//                   column tile records (<= 16 routes of one expert each, with the
//                   token of every route slot)
//                   (reference role: moe.py:504-735, without padding rows)
//                   Up to kFusedTokens tokens, 1 and 2 run as one workgroup
//                   (k_route_sort) with the picks kept in LDS.
//   3. gate/up      per (tile, 16 gate rows): gathered exact MFMA GEMV over the
//                   tile's tokens (quants as fp16 integers, group scale and bias
//                   applied in fp32), h = silu(G_e x) * (U_e x) stored fp32 per
//                   sorted route
//                   (reference role: moe.py:82-135, 225-306; fused rows [0:I] gate,
//                   [I:2I] up, packages/alloy-server/src/alloy_server/models/qwen3_5.py:383-385)
//   4. down         per (tile, 16 hidden rows): D_e h -> fp32 partial per sorted route
//                   (h enters the MFMA as fp16 after a per-token power-of-two scale)
//                   3 and 4 run on the x-stationary kernel (xs.h) when H and I are
//                   multiples of 256 and the group size a power of two (GGUF experts:
//                   always); otherwise MLX experts run k_gate_up / k_down below, which
//                   keep h in fp16.
//   5. k_combine    y[t] = sum_s w[t,s] * partial[inv[t,s]] in slot order
//                   (reference role: moe.py:479-501, fixed-order combine)
// Each expert's weights are read once per column tile of its routed tokens.
#include "gemv.h"
#include "moe.h"
#include "xs.h"

namespace alloy {

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

MoeLayout moe_layout(int64_t T, int E, int top_k, int64_t H, int64_t I) {
  MoeLayout L;
  L.R = T * top_k;
  L.max_tiles = (L.R < E ? L.R : E) + (L.R + kMoeColTile - 1) / kMoeColTile;
  size_t o = 0;
  L.idx = o; o = align256(o + 4 * (size_t)L.R);
  L.wts = o; o = align256(o + 4 * (size_t)L.R);
  L.sorted = o; o = align256(o + 4 * (size_t)L.R);
  L.inv = o; o = align256(o + 4 * (size_t)L.R);
  L.tiles = o; o = align256(o + 4 * kTileInts * (size_t)L.max_tiles);
  L.ntiles = o; o = align256(o + 4);
  L.h = o; o = align256(o + 8 * (size_t)L.R * (size_t)I);   // f32[R][I] (f32[R][2I] routed path)
  L.part = o; o = align256(o + 4 * (size_t)L.R * (size_t)H);
  L.total = o;
  return L;
}

// ------------------------------------------------------------------ router
// One wave routes token t: top-k of the E logits (ties -> lowest index, NaN never
// wins over a number), then the softmax over the k picks in pick order.  Pick k's
// value and index end in lane k; lanes < k write idx / wts (and ridx, when given).
// Each pick is a wave arg-max under the total order (value desc, index asc) by DPP
// row operations (quad swaps, row mirrors, row broadcasts) ending in lane 63, then
// read back as a uniform value — no LDS round trips.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void argmax_dpp(float& bv, int& bi) {
  const int vb = __builtin_bit_cast(int, bv);
  const float ov = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(vb, vb, CTRL, ROW_MASK, 0xF, false));
  const int oi = __builtin_amdgcn_update_dpp(bi, bi, CTRL, ROW_MASK, 0xF, false);
  if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}
__device__ __forceinline__ void wave_argmax(float& bv, int& bi) {
  argmax_dpp<0xB1, 0xF>(bv, bi);    // quad_perm [1,0,3,2]
  argmax_dpp<0x4E, 0xF>(bv, bi);    // quad_perm [2,3,0,1]
  argmax_dpp<0x141, 0xF>(bv, bi);   // row_half_mirror
  argmax_dpp<0x140, 0xF>(bv, bi);   // row_mirror: every lane holds its row's best
  argmax_dpp<0x142, 0xA>(bv, bi);   // row_bcast:15 -> rows 1, 3
  argmax_dpp<0x143, 0xC>(bv, bi);   // row_bcast:31 -> rows 2, 3; lane 63 holds the best
  bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, bv), 63));
  bi = __builtin_amdgcn_readlane(bi, 63);
}
template <int VPL>
__device__ __forceinline__ void route_token(const float* logits, int64_t t, int E, int top_k,
                                            int32_t* idx, float* wts, int* ridx) {
  const int lane = threadIdx.x & 63;
  float v[VPL];
  uint32_t used = 0;
#pragma unroll
  for (int j = 0; j < VPL; ++j) {
    const int e = lane + 64 * j;
    float f = -INFINITY;
    if (e < E) {
      f = logits[t * E + e];
      if (f != f) f = -INFINITY;
    } else {
      used |= 1u << j;
    }
    v[j] = f;
  }
  float myv = -INFINITY;
  int myi = 0;
  for (int k = 0; k < top_k; ++k) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
      const int e = lane + 64 * j;
      if (!((used >> j) & 1u) && (v[j] > bv || (v[j] == bv && e < bi))) { bv = v[j]; bi = e; }
    }
    wave_argmax(bv, bi);
    if ((bi & 63) == lane) used |= 1u << (bi >> 6);
    if (lane == k) { myv = bv; myi = bi; }
  }
  const float m0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, myv), 0));
  float sum = 0.f;
  for (int k = 0; k < top_k; ++k)   // pick order
    sum += expf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, myv), k)) - m0);
  if (lane < top_k) {
    if (idx) idx[t * top_k + lane] = myi;
    if (wts) wts[t * top_k + lane] = expf(myv - m0) / sum;
    if (ridx) ridx[t * top_k + lane] = myi;
  }
}

template <int VPL>
__global__ __launch_bounds__(64) void k_router(const float* logits, int32_t* idx, float* wts, int E,
                                               int top_k) {
  route_token<VPL>(logits, blockIdx.x, E, top_k, idx, wts, nullptr);
}

hipError_t launch_router(const float* logits, int32_t* idx, float* w, int64_t T, int E, int top_k,
                         hipStream_t st) {
  const int vpl = (E + 63) / 64;
  dim3 g((unsigned)T), b(64);
  if (vpl <= 2) hipLaunchKernelGGL(k_router<2>, g, b, 0, st, logits, idx, w, E, top_k);
  else if (vpl <= 4) hipLaunchKernelGGL(k_router<4>, g, b, 0, st, logits, idx, w, E, top_k);
  else if (vpl <= 8) hipLaunchKernelGGL(k_router<8>, g, b, 0, st, logits, idx, w, E, top_k);
  else hipLaunchKernelGGL(k_router<16>, g, b, 0, st, logits, idx, w, E, top_k);
  return hipGetLastError();
}

// ------------------------------------------------------------------ sort
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int t = __shfl_up(v, off, 64);
    if (lane >= off) v += t;
  }
  return v;
}

// Exclusive scan of one value per thread over a 1024-thread block; returns the
// exclusive prefix, *total gets the sum.  scratch: >= 16 ints of LDS.
__device__ int block_excl_scan(int v, int* scratch, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int inc = wave_incl_scan(v, lane);
  if (lane == 63) scratch[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    const int s = lane < 16 ? scratch[lane] : 0;
    const int si = wave_incl_scan(s, lane);
    if (lane < 16) scratch[16 + lane] = si - s;   // exclusive wave offsets
    if (lane == 15) scratch[32] = si;
  }
  __syncthreads();
  const int r = scratch[16 + wave] + inc - v;
  *total = scratch[32];
  __syncthreads();
  return r;
}

constexpr int kSortWaves = 16;
constexpr int kFusedTokens = kSortWaves;   // tokens the one-workgroup router + sort takes

// Stable counting sort of the R routes by expert (order within an expert = route
// order) by one 1024-thread workgroup: sorted (position -> route), inv (route ->
// position) and the column tile records (kTileInts ints each, <= 16 routes of one
// expert, token index = route / top_k per slot).  idx may point to LDS or global
// memory.  lds: wcnt[kSortWaves][E] + eoff[E] + etb[E] + 64 scratch ints.
__device__ void sort_routes(const int* idx, int R, int E, int top_k, int* lds, int32_t* sorted,
                            int32_t* inv, int32_t* tiles, int32_t* ntiles) {
  int* wcnt = lds;                        // [w * E + e]
  int* eoff = lds + kSortWaves * E;       // first sorted position of expert e
  int* etb = eoff + E;                    // first tile of expert e
  int* scratch = etb + E;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  for (int i = tid; i < kSortWaves * E; i += 1024) wcnt[i] = 0;
  __syncthreads();
  const int per = (R + kSortWaves - 1) / kSortWaves;
  const int r0 = wave * per < R ? wave * per : R;
  const int r1 = r0 + per < R ? r0 + per : R;
  for (int r = r0 + lane; r < r1; r += 64) atomicAdd(&wcnt[wave * E + idx[r]], 1);
  __syncthreads();
  int tot = 0;
  if (tid < E)
    for (int w = 0; w < kSortWaves; ++w) tot += wcnt[w * E + tid];
  int all;
  const int off = block_excl_scan(tid < E ? tot : 0, scratch, &all);
  int ntot;
  const int tb = block_excl_scan(tid < E ? (tot + kMoeColTile - 1) / kMoeColTile : 0, scratch, &ntot);
  if (tid < E) {
    eoff[tid] = off;
    etb[tid] = tb;
    int base = off;
    for (int w = 0; w < kSortWaves; ++w) {
      const int c = wcnt[w * E + tid];
      wcnt[w * E + tid] = base;
      base += c;
    }
  }
  __syncthreads();
  // stable placement: each wave walks its route range in order, 64 at a time
  const uint64_t lt = (1ull << lane) - 1ull;
  for (int c0 = r0; c0 < r1; c0 += 64) {
    const int r = c0 + lane;
    const bool valid = r < r1;
    const int e = valid ? idx[r] : 0;
    uint64_t peers = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 10; ++b) {
      const bool bit = (e >> b) & 1;
      const uint64_t bb = __ballot(valid && bit);
      peers &= bit ? bb : ~bb;
    }
    if (valid) {
      const int pos = wcnt[wave * E + e] + __popcll(peers & lt);
      sorted[pos] = r;
      inv[r] = pos;
      const int q = pos - eoff[e];
      tiles[kTileInts * (etb[e] + q / kMoeColTile) + 4 + q % kMoeColTile] = r / top_k;
    }
    __builtin_amdgcn_wave_barrier();
    if (valid && (peers >> lane) == 1ull) wcnt[wave * E + e] += __popcll(peers);
    __builtin_amdgcn_wave_barrier();
  }
  if (tid < E) {
    const int n = tot;
    for (int j = 0; kMoeColTile * j < n; ++j) {
      int32_t* tp = tiles + kTileInts * (tb + j);
      tp[0] = tid;
      tp[1] = off + kMoeColTile * j;
      tp[2] = n - kMoeColTile * j < kMoeColTile ? n - kMoeColTile * j : kMoeColTile;
      tp[3] = 0;
    }
  }
  if (tid == 0) *ntiles = ntot;
}

__global__ __launch_bounds__(1024) void k_sort(const int32_t* idx, int R, int E, int top_k, int32_t* sorted,
                                               int32_t* inv, int32_t* tiles, int32_t* ntiles) {
  extern __shared__ int lds[];
  sort_routes(idx, R, E, top_k, lds, sorted, inv, tiles, ntiles);
}

// Router and sort in one workgroup (T <= kFusedTokens): wave w routes token w; the
// expert picks stay in LDS for the sort.
// lds: ridx[R] + the sort's LDS.
template <int VPL>
__global__ __launch_bounds__(1024) void k_route_sort(const float* logits, int64_t T, int E, int top_k,
                                                     int32_t* idx, float* wts, int32_t* sorted,
                                                     int32_t* inv, int32_t* tiles, int32_t* ntiles) {
  extern __shared__ int lds[];
  const int R = (int)T * top_k;
  int* ridx = lds;
  for (int64_t t = threadIdx.x >> 6; t < T; t += kSortWaves) route_token<VPL>(logits, t, E, top_k, idx, wts, ridx);
  __syncthreads();
  sort_routes(ridx, R, E, top_k, lds + ((R + 63) & ~63), sorted, inv, tiles, ntiles);
}

// Router and sort for at most 64 routes of at most 16 tokens (every expert then has
// at most 16 routes, one column tile): wave w routes token w, then wave 0 sorts with
// one route per lane — rank = routes of smaller experts plus earlier routes of the
// same expert, tile = distinct smaller experts — by a loop over the routes' experts
// read back with readlane.  Same outputs as route + sort_routes.
template <int VPL>
__global__ __launch_bounds__(1024) void k_route_sort_small(const float* logits, int64_t T, int E, int top_k,
                                                           int32_t* idx, float* wts, int32_t* sorted, int32_t* inv,
                                                           int32_t* tiles, int32_t* ntiles) {
  __shared__ int ridx[64];
  const int R = (int)T * top_k;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave < T) route_token<VPL>(logits, wave, E, top_k, idx, wts, ridx);
  __syncthreads();
  if (wave != 0) return;
  const bool valid = lane < R;
  const int e = valid ? ridx[lane] : 0x7FFFFFFF;
  int off = 0, cnt = 0, dup = 0;
  for (int j = 0; j < R; ++j) {
    const int ej = __builtin_amdgcn_readlane(e, j);
    off += ej < e ? 1 : 0;                    // routes of smaller experts
    cnt += ej == e ? 1 : 0;
    dup += (ej == e && j < lane) ? 1 : 0;     // earlier routes of the same expert
  }
  const int rank = off + dup, first = dup == 0 ? 1 : 0;   // first: its expert's first route
  int tile = 0, nd = 0;
  for (int j = 0; j < R; ++j) {
    const int fj = __builtin_amdgcn_readlane(first, j);
    tile += (fj && __builtin_amdgcn_readlane(e, j) < e) ? 1 : 0;   // distinct smaller experts
    nd += fj;
  }
  if (valid) {
    sorted[rank] = lane;
    inv[lane] = rank;
    int32_t* tp = tiles + kTileInts * tile;
    tp[4 + (rank - off)] = lane / top_k;
    if (dup == 0) {
      tp[0] = e;
      tp[1] = off;
      tp[2] = cnt;
      tp[3] = 0;
    }
  }
  if (lane == 0) *ntiles = nd;
}

// ------------------------------------------------------------------ grouped GEMVs
__device__ __forceinline__ void dec32_mlx_f16(const QArgs& a, int64_t n, int k0, f16x8 (&o)[4]) {
  float w[32];
  FMLX::dec32(a, n, k0, w);
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[j][e] = (f16)w[8 * j + e];
}

// Fixed-order reduction of per-wave MFMA accumulators through LDS: wave 0 ends with
// acc(w0) + acc(w1) + acc(w2) + acc(w3).
template <int NA>
__device__ __forceinline__ void reduce_waves(f32x4 (&acc)[NA], float (*red)[NA][64][4]) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wave > 0)
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int t = 0; t < 4; ++t) red[wave - 1][a][lane][t] = acc[a][t];
  __syncthreads();
  if (wave == 0)
#pragma unroll
    for (int w = 0; w < 3; ++w)
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[a][t] += red[w][a][lane][t];
}

// Exact grouped MFMA over MLX rows.  A = 16 activation rows (lane % 16), B = 16
// weight rows (lane % 16) whose quants enter as the fp16 integers 1024 + q (exact:
// the nibble is OR-ed into the mantissa of 1024.0), so every product is exact and
// the MFMA sums them in fp32.  Per group g (gs elements, a multiple of 32) with a
// fresh accumulator:  sum_k w x = s*sum q x + b*X = s*D + (b - 1024 s)*X, where
// D = sum (1024 + q) x and X = sum x (the same MFMA against a ones operand).  The
// activations are permuted to the nibble order (e0,e4)(e1,e5)(e2,e6)(e3,e7) that the
// unpack produces.  Groups are dealt round-robin to the 4 waves.
// Result: acc[w][t] = partial of activation row 4*(lane/16)+t times weight row lane%16.
#define MAGIC1024 0x64006400u   // fp16 1024.0 in both halves

template <int NW>
__device__ __forceinline__ void mlx_rows_mfma(const QArgs& a, const int64_t (&row)[NW], bool rin,
                                              const f16* act, bool ain, f32x4 (&acc)[NW]) {
  const int K = a.K, gs = a.gs, G = K / gs;
  const int wave = threadIdx.x >> 6, kq = (threadIdx.x & 63) >> 4;
  const f16x8 ones = {1, 1, 1, 1, 1, 1, 1, 1};
  const uint32_t magic = MAGIC1024;
  for (int g = wave; g < G; g += 4) {
    f32x4 dX = {0.f, 0.f, 0.f, 0.f};
    f32x4 dW[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w) dW[w] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int h = 0; h < gs; h += 32) {
      const int k = g * gs + h + 8 * kq;
      u32x4 xv = ain ? *(const u32x4*)(act + k) : u32x4{0u, 0u, 0u, 0u};
      // (x0,x4) (x1,x5) (x2,x6) (x3,x7)
      const u32x4 xp = {__builtin_amdgcn_perm(xv.z, xv.x, 0x05040100u), __builtin_amdgcn_perm(xv.z, xv.x, 0x07060302u),
                        __builtin_amdgcn_perm(xv.w, xv.y, 0x05040100u), __builtin_amdgcn_perm(xv.w, xv.y, 0x07060302u)};
      const f16x8 af = __builtin_bit_cast(f16x8, xp);
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const uint32_t q = rin ? *(const uint32_t*)(a.w + row[w] * a.rb + (k >> 1)) : 0u;
        // plain expressions, not inline asm: the hazard recognizer must see these VGPR
        // writes, which can land in registers an earlier MFMA is still reading
        const u32x4 bq = {(q & 0x000F000Fu) | magic, ((q >> 4) & 0x000F000Fu) | magic,
                          ((q >> 8) & 0x000F000Fu) | magic, ((q >> 12) & 0x000F000Fu) | magic};
        dW[w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, __builtin_bit_cast(f16x8, bq), dW[w], 0, 0, 0);
      }
      dX = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, ones, dX, 0, 0, 0);
    }
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int64_t gi = row[w] * G + g;
      const float sc = rin ? h2f(a.s[gi]) : 0.f, bi = rin ? h2f(a.b[gi]) : 0.f;
      const float c = bi - 1024.f * sc;
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[w][t] += sc * dW[w][t] + c * dX[t];
    }
  }
}

__global__ __launch_bounds__(256) void k_gate_up(QArgs gu, const f16* x, const int32_t* sorted,
                                                 const int32_t* tiles, const int32_t* ntiles,
                                                 f16* h, int top_k, int I) {
  __shared__ float red[3][2][64][4];
  const int tile = blockIdx.x;
  if (tile >= *ntiles) return;
  const int e = tiles[kTileInts * tile], p0 = tiles[kTileInts * tile + 1], cnt = tiles[kTileInts * tile + 2];
  const int i0 = blockIdx.y * 16;
  const int K = gu.K;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, kq = lane >> 4;
  // A operand: routed token of column slot n; B operand: gate / up row i0 + n
  const bool ain = n < cnt;
  const f16* act = x + (ain ? (int64_t)(sorted[p0 + n] / top_k) * K : 0);
  const bool rin = i0 + n < I;
  const int64_t rg = (int64_t)e * 2 * I + (rin ? i0 + n : 0);
  const int64_t row[2] = {rg, rg + I};
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  mlx_rows_mfma<2>(gu, row, rin, act, ain, acc);
  reduce_waves<2>(acc, red);
  if (wave == 0 && rin) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int m = 4 * kq + t;                 // route slot within the tile
      if (m < cnt) {
        const float g = acc[0][t], u = acc[1][t];
        h[(int64_t)(p0 + m) * I + i0 + n] = (f16)(g / (1.f + expf(-g)) * u);
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_down(QArgs dn, const f16* h, const int32_t* tiles,
                                              const int32_t* ntiles, float* part, int H) {
  __shared__ float red[3][1][64][4];
  const int tile = blockIdx.x;
  if (tile >= *ntiles) return;
  const int e = tiles[kTileInts * tile], p0 = tiles[kTileInts * tile + 1], cnt = tiles[kTileInts * tile + 2];
  const int j0 = blockIdx.y * 16;
  const int K = dn.K;   // = I
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int n = lane & 15, kq = lane >> 4;
  const bool ain = n < cnt;
  const f16* act = h + (ain ? (int64_t)(p0 + n) * K : 0);
  const bool rin = j0 + n < H;
  const int64_t row[1] = {(int64_t)e * H + (rin ? j0 + n : 0)};
  f32x4 acc[1] = {f32x4{0.f, 0.f, 0.f, 0.f}};
  mlx_rows_mfma<1>(dn, row, rin, act, ain, acc);
  reduce_waves<1>(acc, red);
  if (wave == 0 && rin) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int m = 4 * kq + t;
      if (m < cnt) part[(int64_t)(p0 + m) * H + j0 + n] = acc[0][t];
    }
  }
}

// Slots in groups of 8: the group's weights and partials are all requested before
// the first is added (a loop that adds each slot as it arrives waits one memory
// latency per slot), then summed in slot order.
__global__ __launch_bounds__(256) void k_combine(const float* part, const int32_t* inv,
                                                 const float* wts, float* y, int top_k, int H) {
  constexpr int G = 8;
  const int64_t t = blockIdx.x;
  const int j = blockIdx.y * 256 + threadIdx.x;
  if (j >= H) return;
  float acc = 0.f;
  for (int s0 = 0; s0 < top_k; s0 += G) {
    float w[G], p[G];
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int64_t r = t * top_k + s0 + i;
      const bool in = s0 + i < top_k;
      w[i] = in ? wts[r] : 0.f;
      p[i] = in ? part[(int64_t)(inv ? inv[r] : r) * H + j] : 0.f;   // no inv: partials in route order
    }
#pragma unroll
    for (int i = 0; i < G; ++i)
      if (s0 + i < top_k) acc += w[i] * p[i];
  }
  y[t * H + j] = acc;
}

// gate/up and down on the x-stationary kernel (K of both a multiple of 256, group
// size a power of two); hipErrorNotSupported otherwise, before anything is launched.
template <int GSH>
static hipError_t experts_xs(const MoeArgs& m, const MoeLayout& L, const int32_t* sorted,
                             const int32_t* tiles, const int32_t* ntiles, float* h, float* part,
                             hipStream_t st) {
  XsJob g{};
  g.a = m.gu;
  g.sb = (uint32_t)(m.H / m.gu.gs * 2);
  g.x = m.x;
  g.xbytes = (uint32_t)(m.T * m.H * 2);
  g.xld = (int)m.H;
  g.M = (int)(m.T < 16 ? m.T : 16);   // routes per tile <= tokens
  g.N = (int)m.I;
  g.tiles = tiles;
  g.ntiles = ntiles;
  g.h = h;
  XsJob d = g;
  d.a = m.dn;
  d.sb = (uint32_t)(m.I / m.dn.gs * 2);
  d.x = h;
  d.xbytes = (uint32_t)(L.R * m.I * 4);
  d.xld = (int)m.I;
  d.N = (int)m.H;
  d.part = part;
  // weights dequantised to fp16 with 16-byte loads (fewer load instructions: the
  // grouped kernels are address-unit bound; measured 172 -> 157 us at T = 256)
  hipError_t e = launch_xs<XsMLXD<GSH>, 1>(g, L.max_tiles, 0, 0, st);
  if (e != hipSuccess) return e;
  e = launch_xs<XsMLXD<GSH>, 2>(d, L.max_tiles, 0, 0, st);
  // the gate/up launch has been enqueued: a down launch that does not fit is an error
  return e == hipErrorNotSupported ? hipErrorInvalidValue : e;
}

static hipError_t launch_experts_xs(const MoeArgs& m, const MoeLayout& L, const int32_t* sorted,
                                    const int32_t* tiles, const int32_t* ntiles, float* h, float* part,
                                    hipStream_t st) {
  const int gs = m.gu.gs;
  if (m.H % 256 || m.I % 256 || m.H > 4096 || m.I > 8192 || (gs & (gs - 1)) || gs < 32 || gs > 4096 ||
      L.max_tiles > 65535 || (uint64_t)m.T * m.H * 2 >= (1ull << 31) || (uint64_t)L.R * m.I * 4 >= (1ull << 31) ||
      (uint64_t)(2 * m.I + 16) * m.gu.rb >= (1ull << 31) || (uint64_t)(m.H + 16) * m.dn.rb >= (1ull << 31))
    return hipErrorNotSupported;
  switch (gs) {
    case 32: return experts_xs<0>(m, L, sorted, tiles, ntiles, h, part, st);
    case 64: return experts_xs<1>(m, L, sorted, tiles, ntiles, h, part, st);
    case 128: return experts_xs<2>(m, L, sorted, tiles, ntiles, h, part, st);
    case 256: return experts_xs<3>(m, L, sorted, tiles, ntiles, h, part, st);
    case 512: return experts_xs<4>(m, L, sorted, tiles, ntiles, h, part, st);
    case 1024: return experts_xs<5>(m, L, sorted, tiles, ntiles, h, part, st);
    case 2048: return experts_xs<6>(m, L, sorted, tiles, ntiles, h, part, st);
    default: return experts_xs<7>(m, L, sorted, tiles, ntiles, h, part, st);
  }
}

// Router + sort (one fused workgroup for small batches) into the workspace.
static hipError_t route_and_sort(const MoeArgs& m, const MoeLayout& L, hipStream_t st) {
  int32_t* idx = (int32_t*)(m.ws + L.idx);
  float* wts = (float*)(m.ws + L.wts);
  int32_t* sorted = (int32_t*)(m.ws + L.sorted);
  int32_t* inv = (int32_t*)(m.ws + L.inv);
  int32_t* tiles = (int32_t*)(m.ws + L.tiles);
  int32_t* ntiles = (int32_t*)(m.ws + L.ntiles);
  hipError_t e = hipSuccess;
  const size_t sort_lds = (size_t)(kSortWaves * m.E + 2 * m.E + 64) * sizeof(int);
  if (L.R <= 64 && m.T <= kMoeColTile) {
    const int vpl = (m.E + 63) / 64;
    const dim3 g(1), b((unsigned)(64 * m.T));
    if (vpl <= 2)
      hipLaunchKernelGGL(k_route_sort_small<2>, g, b, 0, st, m.logits, m.T, m.E, m.top_k, idx, wts, sorted, inv, tiles, ntiles);
    else if (vpl <= 4)
      hipLaunchKernelGGL(k_route_sort_small<4>, g, b, 0, st, m.logits, m.T, m.E, m.top_k, idx, wts, sorted, inv, tiles, ntiles);
    else if (vpl <= 8)
      hipLaunchKernelGGL(k_route_sort_small<8>, g, b, 0, st, m.logits, m.T, m.E, m.top_k, idx, wts, sorted, inv, tiles, ntiles);
    else
      hipLaunchKernelGGL(k_route_sort_small<16>, g, b, 0, st, m.logits, m.T, m.E, m.top_k, idx, wts, sorted, inv, tiles, ntiles);
    return hipGetLastError();
  }
  if (m.T <= kFusedTokens) {
    const size_t shm = sort_lds + (size_t)((L.R + 63) & ~63) * sizeof(int);
    auto fused = [&](auto kern) -> hipError_t {
      if (shm > 65536) {
        const hipError_t r = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm);
        if (r != hipSuccess) return r;
      }
      hipLaunchKernelGGL(kern, dim3(1), dim3(1024), shm, st, m.logits, m.T, m.E, m.top_k, idx, wts, sorted, inv,
                         tiles, ntiles);
      return hipGetLastError();
    };
    const int vpl = (m.E + 63) / 64;
    return vpl <= 2 ? fused(k_route_sort<2>) : vpl <= 4 ? fused(k_route_sort<4>)
         : vpl <= 8 ? fused(k_route_sort<8>) : fused(k_route_sort<16>);
  }
  e = launch_router(m.logits, idx, wts, m.T, m.E, m.top_k, st);
  if (e != hipSuccess) return e;
  if (sort_lds > 65536) {
    e = hipFuncSetAttribute((const void*)k_sort, hipFuncAttributeMaxDynamicSharedMemorySize, (int)sort_lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(k_sort, dim3(1), dim3(1024), sort_lds, st, idx, (int)L.R, m.E, m.top_k, sorted, inv, tiles,
                     ntiles);
  return hipGetLastError();
}

static hipError_t combine(const MoeArgs& m, const MoeLayout& L, hipStream_t st) {
  hipLaunchKernelGGL(k_combine, dim3((unsigned)m.T, (unsigned)((m.H + 255) / 256)), dim3(256), 0, st,
                     (const float*)(m.ws + L.part), (const int32_t*)(m.ws + L.inv), (const float*)(m.ws + L.wts),
                     m.y, m.top_k, (int)m.H);
  return hipGetLastError();
}

// ------------------------------------------------------------------ routed wave GEMV (few tokens)
// For T <= kRoutedTokens each route slot r (token r / top_k, expert idx[r]) is one
// GEMV over its expert's rows, on the lane / unit layout of the dense wave-row GEMV
// (k_gemv_w): L lanes per row, <= 4 units per lane with their x in registers, a
// one-row register ring of weights, DPP row sums.  The workgroup's expert is read on
// the device (blockIdx.x = slot * gx + row group).  MODE 0 (gate/up): x = the slot's
// token row, y = fp32 rows [0, 2I) of the slot.  MODE 1 (down): x = silu(g) * u of
// the slot's fp32 gate/up row, scaled by a power of two so its largest magnitude lands
// in [2^14, 2^15) before the fp16 rounding; the sums are scaled back on the store.
constexpr int kRoutedTokens = 16;

template <class F, int UPT, int MODE, int VPL>
// (arguments as scalars, the first dependent loads' inputs first: the dispatch preloads
// the leading ones into SGPRs)
__global__ __launch_bounds__(256) void k_gemv_routed(const float* logits, int gx, int E, int top_k, int lshift,
                                                     const uint8_t* aw, const uint16_t* as, const uint16_t* ab,
                                                     int64_t arb, int aK, int N, uint32_t sb, const void* xsrc,
                                                     float* ys, int32_t* idx, float* wts, const uint8_t* aaux,
                                                     int ags) {
  QArgs a{aw, aaux, as, ab, arb, ags, aK};
  const int r = (int)blockIdx.x / gx, bx = (int)blockIdx.x - r * gx;
  int e;
  if constexpr (VPL > 0) {
    // the router runs here (wave 0 routes the slot's token; the token's first
    // workgroup stores idx / wts for the later launches): no separate launch
    __shared__ int picks[64];
    const int tk = r / top_k;
    if (threadIdx.x < 64) {
      const bool store = bx == 0 && r % top_k == 0;
      route_token<VPL>(logits + (int64_t)tk * E, 0, E, top_k, store ? idx + tk * top_k : nullptr,
                       store ? wts + tk * top_k : nullptr, picks);
    }
    __syncthreads();
    e = __builtin_amdgcn_readfirstlane(picks[r % top_k]);
  } else {
    e = __builtin_amdgcn_readfirstlane(idx[r]);
  }
  const int64_t row0 = (int64_t)e * N;               // the expert's first row
  a.w += row0 * a.rb;
  if (a.s) a.s += row0 * (sb / 2);
  if (a.b) a.b += row0 * (sb / 2);
  const int L = 1 << lshift;
  const int t = threadIdx.x, li = t & (L - 1), slot = t >> lshift;
  const int R = blockDim.x >> lshift;
  const int K = a.K, U = K / F::UE;
  const uint32_t rb = (uint32_t)a.rb;
  const Src src(a, (uint32_t)N * rb, (uint32_t)N * sb);
  const __amdgpu_buffer_rsrc_t yr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(ys + (int64_t)r * N), (short)0, (int)((uint32_t)N * 4u), ALLOY_RSRC_DW3);
  bool own[UPT];
  int uu[UPT];
  uint32_t wo[UPT], so[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) {
    const int u = li + L * j;
    own[j] = u < U;
    uu[j] = own[j] ? u : U - 1;
    wo[j] = own[j] ? F::woff(a, uu[j]) : 0x80000000u;
    so[j] = own[j] ? F::soff(a, uu[j]) : 0x80000000u;
  }
  const int stride = gx * R;
  const int n0 = bx * R + slot;
  uint32_t rw = (uint32_t)n0 * rb, rs = (uint32_t)n0 * sb;
  const uint32_t dw = (uint32_t)stride * rb, ds = (uint32_t)stride * sb;

  constexpr int XV = 512 * F::UE / 4096;             // 16-byte chunks per thread at the largest K
  __shared__ __attribute__((aligned(16))) f16 xl[256 * F::UE];
  __shared__ float wmax[4];
  float yscale = 1.f;
  u32x4 xv[XV], uv[XV];
  const uint32_t xbytes = (MODE == 0 ? 2u : 4u) * (uint32_t)K;   // one activation / gate row
  if constexpr (MODE == 0) {
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const f16*)xsrc + (int64_t)(r / top_k) * K), (short)0, (int)xbytes, ALLOY_RSRC_DW3);
#pragma unroll
    for (int i = 0; i < XV; ++i)
      if (4096u * i < xbytes) xv[i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (uint32_t)t * 16u + 4096u * i, 0, 0);
  } else {
    // gate and up rows of the slot (fp32, K each); thread t holds elements 4t + 1024i
    const float* gu = (const float*)xsrc + (int64_t)r * 2 * K;
    const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc((void*)gu, (short)0, (int)xbytes, ALLOY_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t urs = __builtin_amdgcn_make_buffer_rsrc((void*)(gu + K), (short)0, (int)xbytes, ALLOY_RSRC_DW3);
#pragma unroll
    for (int i = 0; i < XV; ++i)
      if (4096u * i < xbytes) {
        xv[i] = __builtin_amdgcn_raw_buffer_load_b128(grs, (uint32_t)t * 16u + 4096u * i, 0, 0);
        uv[i] = __builtin_amdgcn_raw_buffer_load_b128(urs, (uint32_t)t * 16u + 4096u * i, 0, 0);
      }
  }
  typename F::Raw ring[UPT];
#pragma unroll
  for (int j = 0; j < UPT; ++j) ring[j] = F::load_b(src, rw + wo[j], rs + so[j], uu[j]);
  if constexpr (MODE == 0) {
#pragma unroll
    for (int i = 0; i < XV; ++i)
      if (4096u * i < xbytes) *(u32x4*)((uint8_t*)xl + t * 16 + 4096 * i) = xv[i];
  } else {
    float hv[XV][4];
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      if (4096u * i >= xbytes) break;                   // chunks past the row were not loaded
      const uint32_t g0 = xv[i].x, g1 = xv[i].y, g2 = xv[i].z, g3 = xv[i].w;   // scalars first
      const uint32_t u0 = uv[i].x, u1 = uv[i].y, u2 = uv[i].z, u3 = uv[i].w;
      const uint32_t gb[4] = {g0, g1, g2, g3}, ub[4] = {u0, u1, u2, u3};
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float g = __builtin_bit_cast(float, gb[q]), u = __builtin_bit_cast(float, ub[q]);
        const float h = g / (1.f + __expf(-g)) * u;
        hv[i][q] = h;
        mx = fmaxf(mx, fabsf(h));
      }
    }
    // workgroup max |h| (fixed-shape reduction; max is order independent)
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if ((t & 63) == 0) wmax[t >> 6] = mx;
    lds_barrier_asm();
    mx = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int ex = 0;
    (void)frexpf(mx, &ex);                              // mx = f * 2^ex, f in [0.5, 1)
    const float xs = (mx > 0.f && mx < INFINITY) ? ldexpf(1.f, 15 - ex) : 1.f;
    yscale = 1.f / xs;                                  // exact: a power of two
#pragma unroll
    for (int i = 0; i < XV; ++i)
      if (4096u * i < xbytes) {
        const f16x4 hh = f16x4{(f16)(hv[i][0] * xs), (f16)(hv[i][1] * xs), (f16)(hv[i][2] * xs), (f16)(hv[i][3] * xs)};
        *(f16x4*)((uint8_t*)xl + t * 8 + 2048 * i) = hh;
      }
  }
  lds_barrier_asm();
  uint32_t xr[UPT][F::UE / 2];
  float xg[UPT][F::UE / 16];
#pragma unroll
  for (int j = 0; j < UPT; ++j) load_x_unit<F, f16>(xl, uu[j], xr[j], xg[j]);

  for (int nb = bx * R; nb < N; nb += stride) {        // uniform across the workgroup
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < UPT; ++j) {
      if constexpr (HasShare<F>::value) F::share(ring[j]);
      const float v = F::dot(ring[j], uu[j], xr[j], xg[j]);
      acc += own[j] ? v : 0.f;
    }
    rw += dw;
    rs += ds;
#pragma unroll
    for (int j = 0; j < UPT; ++j) ring[j] = F::load_b(src, rw + wo[j], rs + so[j], uu[j]);
    acc = dpp_sum_rows(acc, lshift) * yscale;
    const uint32_t yo = li == L - 1 ? (uint32_t)(nb + slot) * 4u : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, acc), yr, yo, 0, 0);
  }
}

template <class F, int MODE>
static hipError_t launch_routed(const QArgs& a, uint32_t sb, int32_t* idx, float* wts, const float* logits, int E,
                                int top_k, const void* xsrc, int N, float* ys, int64_t R, hipStream_t st) {
  const int U = a.K / F::UE;
  if (a.K % 256 || U > 256 || (MODE == 1 && a.K > 4096)) return hipErrorNotSupported;
  int lshift = U <= 64 ? 4 : U <= 128 ? 5 : 6;
  const int cus = cu_count();
  while (lshift < 6 && R * ((int64_t)N << lshift) < (int64_t)2 * cus * 256) ++lshift;   // enough workgroups
  const int L = 1 << lshift, upt = (U + L - 1) / L, rows = 256 >> lshift;
  if (upt > 4) return hipErrorNotSupported;
  int64_t gx = (N + rows - 1) / rows;
  const int64_t cap = (3 * (int64_t)cus + R - 1) / R;
  if (gx > cap) gx = cap;
  const dim3 grid((unsigned)(R * gx)), block(256);
  // logits given: the router is fused in (E <= 128 or <= 256 experts); else idx is read
  const int vpl = logits ? (E <= 128 ? 2 : E <= 256 ? 4 : -1) : 0;
  if (vpl < 0) return hipErrorNotSupported;
  auto go = [&](auto u, auto v) {
    constexpr int UP = decltype(u)::value, VP = decltype(v)::value;
    hipLaunchKernelGGL((k_gemv_routed<F, UP, MODE, VP>), grid, block, 0, st, logits, (int)gx, E, top_k, lshift, a.w, a.s,
                       a.b, a.rb, a.K, N, sb, xsrc, ys, idx, wts, a.aux, a.gs);
    return hipGetLastError();
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  using I4 = std::integral_constant<int, 4>;
  using V0 = std::integral_constant<int, 0>;
  if constexpr (MODE == 0) {
    if (vpl == 2) return upt == 1 ? go(I1(), I2()) : upt == 2 ? go(I2(), I2()) : upt == 3 ? go(I3(), I2()) : go(I4(), I2());
    if (vpl == 4) return upt == 1 ? go(I1(), I4()) : upt == 2 ? go(I2(), I4()) : upt == 3 ? go(I3(), I4()) : go(I4(), I4());
  }
  return upt == 1 ? go(I1(), V0()) : upt == 2 ? go(I2(), V0()) : upt == 3 ? go(I3(), V0()) : go(I4(), V0());
}

// Few tokens: gate/up with the router fused in (2I rows of each slot's expert), down
// (H rows over silu(g)*u), combine over the slots in route order: three launches.
template <class FG, class FD>
static hipError_t routed_moe(const MoeArgs& m, const MoeLayout& L, uint32_t sbg, uint32_t sbd, hipStream_t st) {
  int32_t* idx = (int32_t*)(m.ws + L.idx);
  float* wts = (float*)(m.ws + L.wts);
  float* gu = (float*)(m.ws + L.h);
  float* part = (float*)(m.ws + L.part);
  hipError_t e = launch_routed<FG, 0>(m.gu, sbg, idx, wts, m.logits, m.E, m.top_k, m.x, (int)(2 * m.I), gu, L.R, st);
  if (e == hipErrorNotSupported) {            // many experts: a separate router launch
    (void)hipGetLastError();
    if ((e = launch_router(m.logits, idx, wts, m.T, m.E, m.top_k, st)) != hipSuccess) return e;
    e = launch_routed<FG, 0>(m.gu, sbg, idx, wts, nullptr, m.E, m.top_k, m.x, (int)(2 * m.I), gu, L.R, st);
  }
  if (e != hipSuccess) return e;
  if ((e = launch_routed<FD, 1>(m.dn, sbd, idx, wts, nullptr, m.E, m.top_k, gu, (int)m.H, part, L.R, st)) != hipSuccess)
    return e;
  hipLaunchKernelGGL(k_combine, dim3((unsigned)m.T, (unsigned)((m.H + 255) / 256)), dim3(256), 0, st,
                     (const float*)part, (const int32_t*)nullptr, (const float*)wts, m.y, m.top_k, (int)m.H);
  return hipGetLastError();
}

static bool routed_fits(const MoeArgs& m) {
  // 32-bit offsets within one expert; gate/up K = H and down K = I multiples of 256
  return m.T <= kRoutedTokens && m.H % 256 == 0 && m.I % 256 == 0 && m.H <= 8192 && m.I <= 4096 &&
         (uint64_t)(2 * m.I + 256) * (uint64_t)m.gu.rb < (1ull << 31) && (uint64_t)(m.H + 256) * (uint64_t)m.dn.rb < (1ull << 31);
}

hipError_t launch_mlx_moe(const MoeArgs& m, const MoeLayout& L, hipStream_t st) {
  if (routed_fits(m) && m.gu.gs >= 32 && m.dn.gs >= 32) {
    const hipError_t r = routed_moe<FMLX, FMLX>(m, L, 2u * (uint32_t)(m.H / m.gu.gs), 2u * (uint32_t)(m.I / m.dn.gs), st);
    if (r != hipErrorNotSupported) return r;
    (void)hipGetLastError();
  }
  int32_t* sorted = (int32_t*)(m.ws + L.sorted);
  int32_t* tiles = (int32_t*)(m.ws + L.tiles);
  int32_t* ntiles = (int32_t*)(m.ws + L.ntiles);
  float* part = (float*)(m.ws + L.part);
  hipError_t e = route_and_sort(m, L, st);
  if (e != hipSuccess) return e;
  e = launch_experts_xs(m, L, sorted, tiles, ntiles, (float*)(m.ws + L.h), part, st);
  if (e == hipErrorNotSupported) {
    (void)hipGetLastError();
    f16* h16 = (f16*)(m.ws + L.h);             // this pair keeps h in fp16
    hipLaunchKernelGGL(k_gate_up, dim3((unsigned)L.max_tiles, (unsigned)((m.I + 15) / 16)), dim3(256), 0, st,
                       m.gu, m.x, sorted, tiles, ntiles, h16, m.top_k, (int)m.I);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_down, dim3((unsigned)L.max_tiles, (unsigned)((m.H + 15) / 16)), dim3(256), 0, st,
                       m.dn, h16, tiles, ntiles, part, (int)m.H);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  return combine(m, L, st);
}

bool gguf_moe_supported(int64_t T, int64_t H, int64_t I, const MoeLayout& L) {
  // gate/up: two Q4_K matrices of K = H on 8-slot waves (H <= 4096); down: Q6_K of
  // K = I on 8-slot waves (I <= 4096); 32-bit offsets within one expert and in the
  // activation / h buffers
  return H % 256 == 0 && I % 256 == 0 && H <= 4096 && I <= 4096 && L.max_tiles <= 65535 &&
         (uint64_t)T * H * 2 < (1ull << 31) && (uint64_t)L.R * I * 4 < (1ull << 31) &&
         (uint64_t)(2 * I + 16) * (H / 256 * 144) < (1ull << 31) && (uint64_t)(H + 16) * (I / 256 * 210) < (1ull << 31);
}

hipError_t launch_gguf_moe(const MoeArgs& m, const MoeLayout& L, hipStream_t st) {
  if (!gguf_moe_supported(m.T, m.H, m.I, L)) return hipErrorNotSupported;
  if (routed_fits(m)) {
    const hipError_t r = routed_moe<FQ4K, FQ6K>(m, L, 0u, 0u, st);
    if (r != hipErrorNotSupported) return r;
    (void)hipGetLastError();
  }
  hipError_t e = route_and_sort(m, L, st);
  if (e != hipSuccess) return e;
  XsJob g{};
  g.a = m.gu;
  g.x = m.x;
  g.xbytes = (uint32_t)(m.T * m.H * 2);
  g.xld = (int)m.H;
  g.M = (int)(m.T < 16 ? m.T : 16);
  g.N = (int)m.I;
  g.tiles = (const int32_t*)(m.ws + L.tiles);
  g.ntiles = (const int32_t*)(m.ws + L.ntiles);
  g.h = (float*)(m.ws + L.h);
  XsJob d = g;
  d.a = m.dn;
  d.x = g.h;
  d.xbytes = (uint32_t)(L.R * m.I * 4);
  d.xld = (int)m.I;
  d.N = (int)m.H;
  d.part = (float*)(m.ws + L.part);
  // weights dequantised to fp16 before the MFMA (measured 231 -> 221 us at T = 256)
  e = launch_xs<XsDQ<XsQ4K>, 1>(g, L.max_tiles, 0, 0, st);
  if (e != hipSuccess) return e == hipErrorNotSupported ? hipErrorInvalidValue : e;
  // the wire-block Q6_K provider (T = 256: 305 -> 291 us against the word-load one)
  e = launch_xs<XsDQ<XsQ6KW>, 2>(d, L.max_tiles, 0, 0, st);
  if (e != hipSuccess) return e == hipErrorNotSupported ? hipErrorInvalidValue : e;
  return combine(m, L, st);
}

}  // namespace alloy
