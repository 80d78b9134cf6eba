// Block decoders for the quantized-weight formats, written for gfx950 (wave64).
//
// Each format is a struct with three device entry points:
//   dec32(a, n, k0, w[32])   exact fp32 weights of elements k0..k0+31 of row n
//                            (k0 % 32 == 0); every product below is exact in fp32,
//                            so Q8_0/Q5_0/Q6_K are exact and Q4_K/MLX are rounded
//                            once — the values are bit-identical to the reference's
//                            fp32 decode whatever the operation order.
//   load(a, n, u) -> Raw     the raw bytes of decode unit u of row n (registers)
//   dot(raw, xr, xs16)       sum_e w_e * x_e over that unit, for the M=1 GEMV.
//                            Quants are turned into fp16 "1 + q/2^b" values by
//                            placing the b-bit quant in the top mantissa bits of
//                            0x3C00 (exact), dotted with x by v_dot2_f32_f16
//                            (products exact, fp32 accumulation); the 1.0 bias is
//                            removed with the per-16-element x sums xs16.  xr holds
//                            the unit's x as fp16 pairs in the format's XPERM order,
//                            one RUN-element run after the other (run_start gives
//                            the first element of each run); xs16 its sums per 16.
//   constants QK (block elements), UE (unit elements), XPERM (4 or 8).
//
// Layout citations (reference, read-only):
//   Q8_0  packages/alloy-server/src/alloy_server/gguf/quant.py:497-521
//   Q5_0  packages/alloy-server/src/alloy_server/gguf/quant.py:414-494
//   Q4_K  tests/kernels/test_quant_q4k_native.py:45-70,
//         packages/alloy-metal/src/alloy/std/quant.py:835-884
//   Q6_K  packages/alloy-metal/src/alloy/std/quant.py:1200-1270
//   MLX   packages/alloy-server/src/alloy_server/mlx/quant.py:1-24,
//         packages/alloy-metal/src/alloy/std/quant.py:2486-2488
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Arguments describing one quantized weight matrix (N rows of K elements).
struct QArgs {
  const uint8_t* w;     // GGUF wire blocks | MLX qweight | split qweight
  const uint8_t* aux;   // split Q5_0 qhigh
  const uint16_t* s;    // fp16 bits: MLX scales | split scales
  const uint16_t* b;    // fp16 bits: MLX biases
  int64_t rb;           // bytes per row of w
  int32_t gs;           // MLX group size
  int32_t K;
};

__device__ __forceinline__ float h2f(uint32_t bits) {
  return (float)__builtin_bit_cast(f16, (uint16_t)(bits & 0xFFFFu));
}
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(const u32x4*)p; }
__device__ __forceinline__ uint32_t ldu16(const void* p) { return *(const uint16_t*)p; }

// NW little-endian words starting at a 2-byte-aligned address p.  Reads only bytes
// in [p - 2, p + 4*NW): aligned dword loads plus one u16 load, then v_alignbyte.
template <int NW>
__device__ __forceinline__ void ld_words_a2(const uint8_t* p, uint32_t (&o)[NW]) {
  const uint32_t sh = (uint32_t)((uintptr_t)p & 2);   // byte shift: 0 or 2
  // pointer arithmetic (not an integer round trip) keeps the global address space,
  // so these stay global_load instructions rather than FLAT ones
  const uint32_t* q = (const uint32_t*)(p - sh);
  uint32_t t[NW + 1];
#pragma unroll
  for (int i = 0; i < NW; ++i) t[i] = q[i];
  t[NW] = ldu16(p + 4 * NW - 2);             // top half-word, in bounds either way
#pragma unroll
  for (int i = 0; i < NW; ++i) o[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
}

// fp16 pair constants
#define MAGIC1 0x3C003C00u   // fp16 1.0 in both halves

// Bit-field helpers emitted as single VOP3 instructions (the mask lives in an SGPR,
// the other operands in VGPRs: one constant-bus read, as gfx9 allows).  The plain
// expressions compile to an AND and an OR with a literal per use instead (measured
// on the streaming GEMVs: 2-10 % more instructions).  Inline asm hides these writes
// from the hazard recognizer, so they serve only kernels without MFMAs: the decode
// GEMVs, the tile-staged GEMV and the T = 1 routed GEMV; the MFMA kernels decode
// through plain expressions.
__device__ __forceinline__ uint32_t bfi(uint32_t mask, uint32_t a, uint32_t b) {   // (a & mask) | (b & ~mask)
  uint32_t r;
  asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "s"(mask), "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t mask, uint32_t b) { // (a & mask) | b
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(b));
  return r;
}
template <int SH>
__device__ __forceinline__ uint32_t lshl_or(uint32_t a, uint32_t b) {                // (a << SH) | b
  uint32_t r;
  asm("v_lshl_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "i"(SH), "v"(b));
  return r;
}

// Buffer-resource view of one weight matrix (w, aux, s, b), for the streaming
// GEMV.  Raw buffer loads check the offset against the resource size and return
// zero past the end, so rows beyond N (the prefetch runs ahead of the last row)
// need no clamping and can never fault.  Offsets are 32-bit: the host splits
// matrices of 2 GiB or more into row ranges.
#define ALLOY_RSRC_DW3 0x00020000   // gfx9 buffer descriptor word 3: 32-bit data format
struct Src {
  __amdgpu_buffer_rsrc_t w, aux, s, b;
  __device__ Src() {}
  __device__ Src(const QArgs& a, uint32_t wbytes, uint32_t sbytes) {
    w = __builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, (int)wbytes, ALLOY_RSRC_DW3);
    aux = __builtin_amdgcn_make_buffer_rsrc((void*)a.aux, (short)0, a.aux ? (int)wbytes : 0, ALLOY_RSRC_DW3);
    s = __builtin_amdgcn_make_buffer_rsrc((void*)a.s, (short)0, a.s ? (int)sbytes : 0, ALLOY_RSRC_DW3);
    b = __builtin_amdgcn_make_buffer_rsrc((void*)a.b, (short)0, a.b ? (int)sbytes : 0, ALLOY_RSRC_DW3);
  }
};
// P: cache-policy bits of the load (gfx950: 1 sc0, 2 nt, 16 sc1).  kStream marks a
// load whose bytes no other wave reads again (weights streamed once by the M = 1
// GEMV): non-temporal, so they do not push the shared x vector out of the caches.
constexpr int kStream = 2;
template <int P = 0>
__device__ __forceinline__ u32x4 bld16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, P);
}
template <int P = 0>
__device__ __forceinline__ uint32_t bld4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, P);
}
template <int P = 0>
__device__ __forceinline__ uint32_t bld2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, P);
}
// NW little-endian words at a 2-byte-aligned offset: aligned dword loads plus one
// u16 load, merged with v_alignbyte (same bytes as ld_words_a2).
template <int NW>
__device__ __forceinline__ void bwords_a2(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t (&o)[NW]) {
  const uint32_t sh = off & 2u, base = off - sh;
  uint32_t t[NW + 1];
#pragma unroll
  for (int i = 0; i < NW; ++i) t[i] = bld4(r, base + 4 * i);
  t[NW] = bld2(r, off + 4 * NW - 2);
#pragma unroll
  for (int i = 0; i < NW; ++i) o[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
}

// The four fp16 pairs "1 + q/1024" of the 8 nibbles of v (each nibble shifted to bits
// 0-3 of its half), in the order (byte0 lo, byte2 lo), (byte1 lo, byte3 lo),
// (byte0 hi, byte2 hi), (byte1 hi, byte3 hi).
__device__ __forceinline__ void nib_pairs(uint32_t v, uint32_t magic, uint32_t (&p)[4]) {
  p[0] = bfi(0x000F000Fu, v, magic);
  p[1] = bfi(0x000F000Fu, v >> 8, magic);
  p[2] = bfi(0x000F000Fu, v >> 4, magic);
  p[3] = bfi(0x000F000Fu, v >> 12, magic);
}

// ------------------------------------------------------------------ Q4_K
// 144 B: fp16 d | fp16 dmin | scales[12] | qs[128]; sub-block g (32 el) uses
// get_scale_min_k4(g); element l of g is the low (g even) / high nibble of
// qs[(g/2)*32 + l]; w = d*sc*q - dmin*m.
__device__ __forceinline__ void q4k_scale_min(uint32_t S0, uint32_t S1, uint32_t S2, int g,
                                              uint32_t& sc, uint32_t& m) {
  if (g < 4) {
    sc = (S0 >> (8 * g)) & 63u;
    m = (S1 >> (8 * g)) & 63u;
  } else {
    const int j = 8 * (g - 4);
    sc = ((S2 >> j) & 0xFu) | (((S0 >> (j + 6)) & 3u) << 4);
    m = ((S2 >> (j + 4)) & 0xFu) | (((S1 >> (j + 6)) & 3u) << 4);
  }
}

// Branch-free get_scale_min_k4 for a sub-block index that differs across lanes:
// the bit offsets/widths are precomputed once per lane (Q4kSel), then each block
// costs two selects, four bit-field extracts and two shifts-with-or.
struct Q4kSel {
  uint32_t hi;            // 1 when g >= 4
  uint32_t sc_sh, m_sh;   // offset of the low bits of sc / m
  uint32_t lo_w;          // 6 (g < 4) or 4 (g >= 4)
  uint32_t top_sh, top_w; // offset / width (0 or 2) of the top 2 bits in S0 / S1
  __device__ explicit Q4kSel(int g) {
    hi = g >= 4;
    const int j = 8 * (g & 3);
    sc_sh = hi ? j : 8 * g;
    m_sh = hi ? j + 4 : 8 * g;
    lo_w = hi ? 4 : 6;
    top_sh = j + 6;
    top_w = hi ? 2 : 0;
  }
  __device__ __forceinline__ void get(uint32_t S0, uint32_t S1, uint32_t S2, uint32_t& sc, uint32_t& m) const {
    const uint32_t lsc = hi ? S2 : S0, lm = hi ? S2 : S1;
    sc = lshl_or<4>(__builtin_amdgcn_ubfe(S0, top_sh, top_w), __builtin_amdgcn_ubfe(lsc, sc_sh, lo_w));
    m = lshl_or<4>(__builtin_amdgcn_ubfe(S1, top_sh, top_w), __builtin_amdgcn_ubfe(lm, m_sh, lo_w));
  }
};

struct FQ4K {
  static constexpr int QK = 256, BB = 144, UE = 32, XPERM = 4;

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const uint8_t* blk = a.w + n * a.rb + (int64_t)(k0 >> 8) * BB;
    const int g = (k0 & 255) >> 5;
    const u32x4 h = ld16(blk);
    const float d = h2f(h.x), dmin = h2f(h.x >> 16);
    uint32_t sc, m;
    q4k_scale_min(h.y, h.z, h.w, g, sc, m);
    const float dsc = d * (float)sc, dm = dmin * (float)m;
    const uint8_t* qs = blk + 16 + 32 * (g >> 1);
    const u32x4 q0 = ld16(qs), q1 = ld16(qs + 16);
    const uint32_t words[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const int sh = 4 * (g & 1);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        w[4 * i + b] = dsc * (float)((words[i] >> (8 * b + sh)) & 15u) - dm;
  }

  // unit u = (superblock u/8, quant chunk c = u%8): the 16 bytes qs[16c, 16c+16),
  // i.e. elements l0..l0+15 (l0 = 16*(c%2)) of sub-blocks 2p (low nibbles) and
  // 2p+1 (high nibbles), p = c/2.  Eight consecutive lanes read the eight chunks
  // of one superblock, so each load instruction covers contiguous 128-byte runs.
  // runs (16 elements): 64p + l0 + [0,16) and 64p + 32 + l0 + [0,16).
  static constexpr int RUN = 16;
  struct Raw { u32x4 h, q; };
  __device__ static int run_start(int u, int r) {
    const int c = u & 7;
    return 256 * (u >> 3) + 64 * (c >> 1) + 16 * (c & 1) + 32 * r;
  }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) { return load_row(a.w + n * a.rb, u); }
  // row: the row's bytes (global memory or an LDS tile)
  __device__ static Raw load_row(const uint8_t* row, int u) {
    const uint8_t* blk = row + (u >> 3) * BB;
    return Raw{ld16(blk), ld16(blk + 16 + 16 * (u & 7))};
  }
  // byte offset of unit u's super-block in the row (w) and in the scale row (s: none)
  __device__ static uint32_t woff(const QArgs&, int u) { return (uint32_t)(u >> 3) * BB; }
  __device__ static uint32_t soff(const QArgs&, int) { return 0; }
  // Wave-row GEMV (raw buffer loads): the four lanes of a quad hold four units of the
  // same super-block, so each loads one dword of the 16-byte header (d, dmin, scales)
  // and share() broadcasts the four dwords across the quad — a quarter of the header
  // bytes through the address unit instead of the whole header per lane.
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t, int u) {
    Raw r;
    r.h = u32x4{bld4<kStream>(src.w, wo + 4u * (uint32_t)(u & 3)), 0u, 0u, 0u};
    r.q = bld16<kStream>(src.w, wo + 16 + 16 * (u & 7));
    return r;
  }
  // (every lane of the quad is a valid source, so the moves need no old value)
  __device__ static void share(Raw& r) {
    const int v = (int)r.h.x;
    r.h = u32x4{(uint32_t)__builtin_amdgcn_mov_dpp(v, 0x00, 0xF, 0xF, true),    // quad_perm [0,0,0,0]
                (uint32_t)__builtin_amdgcn_mov_dpp(v, 0x55, 0xF, 0xF, true),    // [1,1,1,1]
                (uint32_t)__builtin_amdgcn_mov_dpp(v, 0xAA, 0xF, 0xF, true),    // [2,2,2,2]
                (uint32_t)__builtin_amdgcn_mov_dpp(v, 0xFF, 0xF, 0xF, true)};   // [3,3,3,3]
  }
  // Quants enter v_dot2 as fp16 mantissa fields of 1.0: a low nibble (bits 0-3 of a
  // half) reads 1 + q/1024, a high nibble (bits 4-7) 1 + q/64, so one v_bfi_b32
  // per pair unpacks them (plus one shift for bytes 1 and 3).  Sub-block A (low
  // nibbles): sum q x = 1024 (SA - XA); sub-block B (high): 64 (SB - XB).
  __device__ static float dot(const Raw& r, int u, const uint32_t* xa, const float* xg) {
    const int p = (u & 7) >> 1;
    const uint32_t words[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t* xb = xa + 8;                 // sub-block B pairs
    const uint32_t magic = MAGIC1;
    float SA = 0.f, SB = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = words[i], v8 = v >> 8;
      SA = dot2(bfi(0x000F000Fu, v, magic), xa[2 * i], SA);        // bytes 0,2 low
      SA = dot2(bfi(0x000F000Fu, v8, magic), xa[2 * i + 1], SA);   // bytes 1,3 low
      SB = dot2(bfi(0x00F000F0u, v, magic), xb[2 * i], SB);        // bytes 0,2 high
      SB = dot2(bfi(0x00F000F0u, v8, magic), xb[2 * i + 1], SB);   // bytes 1,3 high
    }
    const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
    uint32_t scA, mA, scB, mB;
    Q4kSel(2 * p).get(r.h.y, r.h.z, r.h.w, scA, mA);
    Q4kSel(2 * p + 1).get(r.h.y, r.h.z, r.h.w, scB, mB);
    const float cA = 1024.f * d * (float)scA, cB = 64.f * d * (float)scB;
    // w = d sc q - dmin m
    return cA * (SA - xg[0]) + cB * (SB - xg[1]) - dmin * ((float)mA * xg[0] + (float)mB * xg[1]);
  }
  // Wave-row GEMV with units u = lane + L j (L even): lanes 2i and 2i + 1 hold the two
  // halves (elements 0-15, 16-31) of the same sub-block pair (2p, 2p + 1).  They add
  // their sums across the pair (DPP) and each applies one sub-block's scale and min —
  // sub-block u % 8: the even lane 2p (low nibbles), the odd lane 2p + 1 (high) — so
  // the scale work per unit is halved.  xgp[0]: the pair's activation sum of this
  // lane's sub-block (pair_x_sums); units past the row read zero headers and add 0.
  __device__ static float dot_pair(const Raw& r, int u, const uint32_t* xa, const float* xgp, bool odd) {
    const uint32_t words[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t* xb = xa + 8;
    const uint32_t magic = MAGIC1;
    float SA = 0.f, SB = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = words[i], v8 = v >> 8;
      SA = dot2(bfi(0x000F000Fu, v, magic), xa[2 * i], SA);
      SA = dot2(bfi(0x000F000Fu, v8, magic), xa[2 * i + 1], SA);
      SB = dot2(bfi(0x00F000F0u, v, magic), xb[2 * i], SB);
      SB = dot2(bfi(0x00F000F0u, v8, magic), xb[2 * i + 1], SB);
    }
    const float PA = SA + pair_swap(SA), PB = SB + pair_swap(SB);
    const float S = odd ? PB : PA, xs = xgp[0];
    uint32_t sc, m;
    Q4kSel(u & 7).get(r.h.y, r.h.z, r.h.w, sc, m);
    const float d = h2f(r.h.x), dmin = h2f(r.h.x >> 16);
    const float c = (odd ? 64.f : 1024.f) * d * (float)sc;
    return c * (S - xs) - dmin * (float)m * xs;
  }
  // the value of lane l ^ 1 (quad_perm [1,0,3,2])
  __device__ static float pair_swap(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
  }
  // xg of the pair_dot layout: xg[0] = the activation sum of the lane's sub-block
  // (2p for the even lane, 2p + 1 for the odd one) over both halves of the pair
  __device__ static void pair_x_sums(float* xg, bool odd) {
    const float a = xg[0] + pair_swap(xg[0]), b = xg[1] + pair_swap(xg[1]);
    xg[0] = odd ? b : a;
  }
};

// ------------------------------------------------------------------ Q6_K
// 210 B: ql[128] | qh[64] | int8 scales[16] | fp16 d; element e = 128h+32s+l:
// ql byte 64h+32(s&1)+l (nibble shift 4(s>>1)), qh byte 32h+l (shift 2s),
// q = (nib | qh2<<4) - 32, scale 8h+2s+l/16; w = d*sc*q.
struct FQ6K {
  static constexpr int QK = 256, BB = 210, UE = 64, XPERM = 4;
  static constexpr int RUN = 32;        // x run length (elements) of a unit

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const uint8_t* blk = a.w + n * a.rb + (int64_t)(k0 >> 8) * BB;
    const int e = k0 & 255, h = e >> 7, s = (e >> 5) & 3;
    uint32_t ql[8], qh[8];
    ld_words_a2<8>(blk + 64 * h + 32 * (s & 1), ql);
    ld_words_a2<8>(blk + 128 + 32 * h, qh);
    const uint32_t scp = ldu16(blk + 192 + 8 * h + 2 * s);
    const float d = h2f(ldu16(blk + 208));
    const float ds0 = d * (float)(int8_t)(scp & 0xFF), ds1 = d * (float)(int8_t)(scp >> 8);
    const int nsh = 4 * (s >> 1), hsh = 2 * s;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int q = (int)(((ql[i] >> (8 * b + nsh)) & 15u) | (((qh[i] >> (8 * b + hsh)) & 3u) << 4)) - 32;
        w[4 * i + b] = (i < 4 ? ds0 : ds1) * (float)q;
      }
  }

  // unit u = (superblock u/4, half h = (u%4)/2, s0 = u%2): runs of elements
  // 128h+32*s0+l (low nibbles) and 128h+32*(s0+2)+l (high nibbles), l in [0,32).
  struct Raw { uint32_t ql[8], qh[8], scl, sch, d; };
  __device__ static int run_start(int u, int r) {
    return 256 * (u >> 2) + 128 * ((u >> 1) & 1) + 32 * (u & 1) + 64 * r;
  }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) { return load_row(a.w + n * a.rb, u); }
  __device__ static Raw load_row(const uint8_t* row, int u) {
    const int h = (u >> 1) & 1, s0 = u & 1;
    const uint8_t* blk = row + (u >> 2) * BB;
    Raw r;
    ld_words_a2<8>(blk + 64 * h + 32 * s0, r.ql);
    ld_words_a2<8>(blk + 128 + 32 * h, r.qh);
    r.scl = ldu16(blk + 192 + 8 * h + 2 * s0);       // scales (s0, l<16), (s0, l>=16)
    r.sch = ldu16(blk + 192 + 8 * h + 2 * s0 + 4);   // scales (s0+2, ...)
    r.d = ldu16(blk + 208);
    return r;
  }
  __device__ static uint32_t woff(const QArgs&, int u) { return (uint32_t)(u >> 2) * BB; }
  __device__ static uint32_t soff(const QArgs&, int) { return 0; }
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t, int u) {
    const int h = (u >> 1) & 1, s0 = u & 1;
    Raw r;
    bwords_a2<8>(src.w, wo + 64 * h + 32 * s0, r.ql);
    bwords_a2<8>(src.w, wo + 128 + 32 * h, r.qh);
    r.scl = bld2(src.w, wo + 192 + 8 * h + 2 * s0);
    r.sch = bld2(src.w, wo + 196 + 8 * h + 2 * s0);
    r.d = bld2(src.w, wo + 208);
    return r;
  }
  __device__ static float dot(const Raw& r, int u, const uint32_t* xlo, const float* xg) {
    const int c0 = 2 * (u & 1);
    const uint32_t magic = MAGIC1;
    const uint32_t* xhi = xlo + 16;
    float S[4] = {0.f, 0.f, 0.f, 0.f};   // (s0,l<16) (s0,l>=16) (s0+2,l<16) (s0+2,l>=16)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t v = r.ql[i], c = r.qh[i];
      // the nibbles where they lie (bytes 1, 3 moved down by 8), the 2-bit highs moved to
      // sit above them: low-nibble u in mantissa bits 0..5 -> 1 + u/1024, high-nibble u
      // in bits 4..9 -> 1 + u/64 (three shifts per word pair)
      const uint32_t v8 = v >> 8;
      const uint32_t c1 = c << (4 - c0);           // highs of bytes 0, 2 at bits 4-5 / 8-9 (+16)
      const uint32_t c18 = c >> (4 + c0);          // highs of bytes 1, 3 at bits 4-5 / 8-9 (+16)
      const uint32_t p0 = bfi(0x00300030u, c1, bfi(0x000F000Fu, v, magic));
      const uint32_t p1 = bfi(0x00300030u, c18, bfi(0x000F000Fu, v8, magic));
      const uint32_t p2 = bfi(0x03000300u, c1, and_or(v, 0x00F000F0u, magic));
      const uint32_t p3 = bfi(0x03000300u, c18, and_or(v8, 0x00F000F0u, magic));
      const int q = i >> 2;
      S[q] = dot2(p0, xlo[2 * i], S[q]);
      S[q] = dot2(p1, xlo[2 * i + 1], S[q]);
      S[2 + q] = dot2(p2, xhi[2 * i], S[2 + q]);
      S[2 + q] = dot2(p3, xhi[2 * i + 1], S[2 + q]);
    }
    // sum((u-32) x) = 1024 S - 1056 X (low nibbles), 64 S - 96 X (high nibbles)
    float acc = (float)(int8_t)(r.scl & 0xFF) * (1024.f * S[0] - 1056.f * xg[0]);
    acc += (float)(int8_t)(r.scl >> 8) * (1024.f * S[1] - 1056.f * xg[1]);
    acc += (float)(int8_t)(r.sch & 0xFF) * (64.f * S[2] - 96.f * xg[2]);
    acc += (float)(int8_t)(r.sch >> 8) * (64.f * S[3] - 96.f * xg[3]);
    return h2f(r.d) * acc;
  }
};

// ------------------------------------------------------------------ Q8_0 (wire)
// 34 B: fp16 d | int8 qs[32]; w = d*q.
// Sum over 32 int8 weights (words v) of (1 + u/1024) x with u = q + 128: each fp16
// pair is one byte permute of the offset-binary word with the fp16 1.0 pattern.
// Callers take sum(q x) = 1024 S - 1152 X.
__device__ __forceinline__ float q8_words_dot(const uint32_t (&v)[8], const uint32_t* xp, float S) {
  const uint32_t magic = MAGIC1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t o = v[i] ^ 0x80808080u;       // offset binary u = q + 128
    S = dot2(__builtin_amdgcn_perm(magic, o, 0x07020500u), xp[2 * i], S);       // bytes 0, 2
    S = dot2(__builtin_amdgcn_perm(magic, o, 0x07030501u), xp[2 * i + 1], S);   // bytes 1, 3
  }
  return S;
}

struct FQ80 {
  static constexpr int QK = 32, BB = 34, UE = 32, XPERM = 4;
  static constexpr int RUN = 32;        // x run length (elements) of a unit

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const uint8_t* blk = a.w + n * a.rb + (int64_t)(k0 >> 5) * BB;
    uint32_t v[8];
    ld_words_a2<8>(blk + 2, v);
    const float d = h2f(ldu16(blk));
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b) w[4 * i + b] = d * (float)(int8_t)((v[i] >> (8 * b)) & 0xFF);
  }

  struct Raw { uint32_t v[8]; uint32_t d; };
  __device__ static int run_start(int u, int) { return 32 * u; }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) { return load_row(a.w + n * a.rb, u); }
  __device__ static Raw load_row(const uint8_t* row, int u) {
    const uint8_t* blk = row + u * BB;
    Raw r;
    ld_words_a2<8>(blk + 2, r.v);
    r.d = ldu16(blk);
    return r;
  }
  __device__ static uint32_t woff(const QArgs&, int u) { return (uint32_t)u * BB; }
  __device__ static uint32_t soff(const QArgs&, int) { return 0; }
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t, int) {
    Raw r;
    bwords_a2<8>(src.w, wo + 2, r.v);
    r.d = bld2(src.w, wo);
    return r;
  }
  __device__ static float dot(const Raw& r, int, const uint32_t* xp, const float* xg) {
    const float S = q8_words_dot(r.v, xp, 0.f);
    return h2f(r.d) * (1024.f * S - 1152.f * (xg[0] + xg[1]));   // sum((u-128) x)
  }
};

// Q8_0 split layout (reference loader): qweight int8[N,K], scales fp16[N,K/32].
struct FQ80S {
  static constexpr int QK = 32, BB = 32, UE = 32, XPERM = 4;
  static constexpr int RUN = 32;        // x run length (elements) of a unit

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const uint8_t* q = a.w + n * a.rb + k0;
    const u32x4 q0 = ld16(q), q1 = ld16(q + 16);
    const uint32_t v[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
    const float d = h2f(a.s[n * (a.K >> 5) + (k0 >> 5)]);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b) w[4 * i + b] = d * (float)(int8_t)((v[i] >> (8 * b)) & 0xFF);
  }

  struct Raw { uint32_t v[8]; uint32_t d; };
  __device__ static int run_start(int u, int) { return 32 * u; }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) {
    const uint8_t* q = a.w + n * a.rb + 32 * u;
    const u32x4 q0 = ld16(q), q1 = ld16(q + 16);
    return Raw{{q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w}, a.s[n * (a.K >> 5) + u]};
  }
  __device__ static uint32_t woff(const QArgs&, int u) { return 32u * (uint32_t)u; }
  __device__ static uint32_t soff(const QArgs&, int u) { return 2u * (uint32_t)u; }
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t so, int) {
    const u32x4 q0 = bld16(src.w, wo), q1 = bld16(src.w, wo + 16);
    return Raw{{q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w}, bld2(src.s, so)};
  }
  __device__ static float dot(const Raw& r, int, const uint32_t* xp, const float* xg) {
    const float S = q8_words_dot(r.v, xp, 0.f);
    return h2f(r.d) * (1024.f * S - 1152.f * (xg[0] + xg[1]));
  }
};

// ------------------------------------------------------------------ Q5_0 (wire)
// 22 B: fp16 d | u32 qh | qs[16]; element l<16: (qs[l]&15) | bit_l(qh)<<4,
// element l+16: (qs[l]>>4) | bit_{l+16}(qh)<<4; w = (q-16)*d.
struct FQ50 {
  static constexpr int QK = 32, BB = 22, UE = 32, XPERM = 4;
  static constexpr int RUN = 32;        // x run length (elements) of a unit

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const uint8_t* blk = a.w + n * a.rb + (int64_t)(k0 >> 5) * BB;
    uint32_t qh1[1], qs[4];
    ld_words_a2<1>(blk + 2, qh1);
    ld_words_a2<4>(blk + 6, qs);
    const uint32_t qh = qh1[0];
    const float d = h2f(ldu16(blk));
#pragma unroll
    for (int l = 0; l < 16; ++l) {
      const uint32_t byte = (qs[l >> 2] >> (8 * (l & 3))) & 0xFF;
      const int lo = (int)((byte & 15u) | (((qh >> l) & 1u) << 4)) - 16;
      const int hi = (int)((byte >> 4) | (((qh >> (l + 16)) & 1u) << 4)) - 16;
      w[l] = d * (float)lo;
      w[l + 16] = d * (float)hi;
    }
  }

  struct Raw { uint32_t qs[4], qh, d; };
  __device__ static int run_start(int u, int) { return 32 * u; }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) { return load_row(a.w + n * a.rb, u); }
  __device__ static Raw load_row(const uint8_t* row, int u) {
    const uint8_t* blk = row + u * BB;
    Raw r;
    uint32_t qh1[1];
    ld_words_a2<1>(blk + 2, qh1);
    ld_words_a2<4>(blk + 6, r.qs);
    r.qh = qh1[0];
    r.d = ldu16(blk);
    return r;
  }
  __device__ static uint32_t woff(const QArgs&, int u) { return (uint32_t)u * BB; }
  __device__ static uint32_t soff(const QArgs&, int) { return 0; }
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t, int) {
    Raw r;
    uint32_t qh1[1];
    bwords_a2<1>(src.w, wo + 2, qh1);
    bwords_a2<4>(src.w, wo + 6, r.qs);
    r.qh = qh1[0];
    r.d = bld2(src.w, wo);
    return r;
  }
  __device__ static float dot(const Raw& r, int, const uint32_t* xp, const float* xg) {
    const uint32_t qh = r.qh, magic = MAGIC1;
    float SA = 0.f, SB = 0.f;
    // Elements 0..15 (low nibbles): 5-bit u in fp16 mantissa bits 0..4 -> 1 + u/1024;
    // elements 16..31 (high nibbles): u in bits 4..8 -> 1 + u/64.  The nibbles stay
    // where they lie (bytes 1, 3 moved down by 8); the 5th bits of four consecutive
    // elements go to bits 0, 8, 16, 24 by one 24-bit multiply (bit j to bit 8j).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = r.qs[i], v8 = v >> 8;
      const int l = 4 * i;
      const uint32_t sA = (((qh >> l) & 15u) * 0x00204081u) & 0x01010101u;
      const uint32_t sB = (((qh >> (l + 16)) & 15u) * 0x00204081u) & 0x01010101u;
      SA = dot2(bfi(0x00100010u, sA << 4, bfi(0x000F000Fu, v, magic)), xp[2 * i], SA);
      SA = dot2(bfi(0x00100010u, sA >> 4, bfi(0x000F000Fu, v8, magic)), xp[2 * i + 1], SA);
      SB = dot2(bfi(0x01000100u, sB << 8, and_or(v, 0x00F000F0u, magic)), xp[8 + 2 * i], SB);
      SB = dot2(bfi(0x01000100u, sB, and_or(v8, 0x00F000F0u, magic)), xp[8 + 2 * i + 1], SB);
    }
    // sum((u-16) x) = 1024 SA - 1040 X_A + 64 SB - 80 X_B
    return h2f(r.d) * (1024.f * SA - 1040.f * xg[0] + (64.f * SB - 80.f * xg[1]));
  }
};

// Q5_0 split layout (reference loader): qweight u8[N,K/2] K-sequential nibbles,
// qhigh u8[N,K/2] (5th bit of element k in bit 0 / of k+1 in bit 4 of byte k/2),
// scales fp16[N,K/32].  packages/alloy-metal/src/alloy/std/quant.py:1025-1034.
struct FQ50S {
  static constexpr int QK = 32, BB = 16, UE = 32, XPERM = 8;
  static constexpr int RUN = 32;        // x run length (elements) of a unit

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const int64_t off = n * a.rb + (k0 >> 1);
    const u32x4 q = ld16(a.w + off), hq = ld16(a.aux + off);
    const uint32_t qv[4] = {q.x, q.y, q.z, q.w}, hv[4] = {hq.x, hq.y, hq.z, hq.w};
    const float d = h2f(a.s[n * (a.K >> 5) + (k0 >> 5)]);
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const int sh = 8 * ((e >> 1) & 3) + 4 * (e & 1);
      const uint32_t nib = (qv[e >> 3] >> sh) & 15u, hb = (hv[e >> 3] >> sh) & 1u;
      w[e] = d * (float)((int)(nib | (hb << 4)) - 16);
    }
  }

  struct Raw { u32x4 q, hq; uint32_t d; };
  __device__ static int run_start(int u, int) { return 32 * u; }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) {
    const int64_t off = n * a.rb + 16 * u;
    return Raw{ld16(a.w + off), ld16(a.aux + off), a.s[n * (a.K >> 5) + u]};
  }
  __device__ static uint32_t woff(const QArgs&, int u) { return 16u * (uint32_t)u; }
  __device__ static uint32_t soff(const QArgs&, int u) { return 2u * (uint32_t)u; }
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t so, int) {
    return Raw{bld16(src.w, wo), bld16(src.aux, wo), bld2(src.s, so)};
  }
  __device__ static float dot(const Raw& r, int, const uint32_t* xp, const float* xg) {
    const uint32_t qv[4] = {r.q.x, r.q.y, r.q.z, r.q.w}, hv[4] = {r.hq.x, r.hq.y, r.hq.z, r.hq.w};
    const uint32_t magic = MAGIC1;
    float S = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t v = qv[i], c = hv[i];
      S = dot2(bfi(0x02000200u, c << 9, bfi(0x01E001E0u, v << 5, magic)), xp[4 * i], S);
      S = dot2(bfi(0x02000200u, c << 1, bfi(0x01E001E0u, v >> 3, magic)), xp[4 * i + 1], S);
      S = dot2(bfi(0x02000200u, c << 5, bfi(0x01E001E0u, v << 1, magic)), xp[4 * i + 2], S);
      S = dot2(bfi(0x02000200u, c >> 3, bfi(0x01E001E0u, v >> 7, magic)), xp[4 * i + 3], S);
    }
    return h2f(r.d) * (32.f * S - 48.f * (xg[0] + xg[1]));
  }
};

// ------------------------------------------------------------------ MLX 4-bit affine
// qweight u8[N,K/2]: byte k/2 low nibble = element k (even); scales/biases
// fp16[N,K/gs]; w = s*q + b.  Units of 32 elements require gs % 32 == 0.
struct FMLX {
  static constexpr int QK = 32, BB = 16, UE = 32, XPERM = 8;
  static constexpr int RUN = 32;        // x run length (elements) of a unit

  __device__ static void dec32(const QArgs& a, int64_t n, int k0, float (&w)[32]) {
    const u32x4 q = ld16(a.w + n * a.rb + (k0 >> 1));
    const uint32_t v[4] = {q.x, q.y, q.z, q.w};
    const int64_t gi = n * (a.K / a.gs) + k0 / a.gs;
    const float s = h2f(a.s[gi]), b = h2f(a.b[gi]);
#pragma unroll
    for (int e = 0; e < 32; ++e) {
      const uint32_t nib = (v[e >> 3] >> (4 * (e & 7))) & 15u;
      w[e] = s * (float)nib + b;
    }
  }

  struct Raw { u32x4 q; uint32_t s, b; };
  __device__ static int run_start(int u, int) { return 32 * u; }
  __device__ static Raw load(const QArgs& a, int64_t n, int u) {
    const int64_t gi = n * (a.K / a.gs) + (32 * u) / a.gs;
    return Raw{ld16(a.w + n * a.rb + 16 * u), a.s[gi], a.b[gi]};
  }
  __device__ static uint32_t woff(const QArgs&, int u) { return 16u * (uint32_t)u; }
  __device__ static uint32_t soff(const QArgs& a, int u) { return 2u * (uint32_t)((32 * u) / a.gs); }
  __device__ static Raw load_b(const Src& src, uint32_t wo, uint32_t so, int) {
    return Raw{bld16(src.w, wo), bld2(src.s, so), bld2(src.b, so)};
  }
  __device__ static float dot(const Raw& r, int, const uint32_t* xp, const float* xg) {
    const uint32_t v[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
    const uint32_t magic = MAGIC1;
    float S = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t pr[4];
      nib_pairs(v[i], magic, pr);                   // (e0,e4) (e2,e6) (e1,e5) (e3,e7)
      S = dot2(pr[0], xp[4 * i], S);
      S = dot2(pr[1], xp[4 * i + 1], S);
      S = dot2(pr[2], xp[4 * i + 2], S);
      S = dot2(pr[3], xp[4 * i + 3], S);
    }
    const float s1k = 1024.f * h2f(r.s);
    return s1k * S + (h2f(r.b) - s1k) * (xg[0] + xg[1]);           // s sum(q x) + b X
  }
};
