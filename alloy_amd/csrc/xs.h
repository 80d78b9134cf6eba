// x-stationary MFMA GEMV for up to 16 activation rows (decode M <= 16 and the
// routed-expert MoE GEMVs), gfx950.
//
// Each wave owns a fixed range of K and keeps the activations of that range (16
// token rows, zero past the row count) as MFMA A operands in registers for the whole
// kernel; the workgroup's W waves cover all of K for the same 16-row weight tiles and
// are reduced through LDS in a fixed order.  B = 16 weight rows with the quants as
// exact fp16 integers (1024 + q, or 1024 + 16q for a high nibble), so every product
// is exact.  The MFMAs of one scale group ("chain") accumulate D (lane: weight row
// l%16, tokens 4(l/16)+t), which is folded in fp32 as
//     y += s*D + c*X,
// with the group's scale s, offset c (the format's offset minus 1024 s) and X the
// group's activation sum per token, computed once per wave (ones operand) into LDS.
// Every weight byte of a group of tiles is requested before any is used.
//
// Units: 256 elements of a row; a wave owns NS/8 units (8 activation slots each).
#pragma once
#include <type_traits>
#include "gemv.h"
#include "launch.h"

namespace alloy {

constexpr uint32_t kXsMagic = 0x64006400u;     // fp16 1024.0 in both halves

// ---------------------------------------------------------------- format providers
// A provider describes one quantized format to the kernel:
//   Raw, load(src, rw, rs, unit, kq, raw): the lane's bytes of one unit of its row
//       (rw / rs: byte offsets of the row in the weight / scale buffers; kq = lane/16)
//   xload(xr, off, S, kq): the lane's 8 activations for slot S (0..7) of a unit whose
//       first element is at byte `off` of the activation buffer, in the order the
//       unpack produces (A operands); xload32: the same 8 from an fp32 buffer
//   NCH, chain<C>(xu, raw): chain C of the unit: its MFMAs on the unit's activation
//       slots xu[0..7], summed in one accumulator D (all products exact)
//   xsum<C>(xu): the same MFMAs against ones (the per-token activation sums X)
//   sc<C>(raw, s, c): the chain's scale and offset: the chain contributes s D + c X.
//   WIDE: whether 16 activation slots per wave (K up to 8192) or two tiles per
//       reduction fit the registers.

// 8 fp16 activations at byte `off` in the order (0,2,1,3, 4,6,5,7)
__device__ __forceinline__ f16x8 xs_x8_perm4(__amdgpu_buffer_rsrc_t xr, uint32_t off) {
  const u32x4 v = bld16(xr, off);
  return __builtin_bit_cast(f16x8, u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                                         __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)});
}
// 8 fp16 activations at byte `off` in the order (0,4,1,5,2,6,3,7)
__device__ __forceinline__ f16x8 xs_x8_perm8(__amdgpu_buffer_rsrc_t xr, uint32_t off) {
  const u32x4 v = bld16(xr, off);
  return __builtin_bit_cast(f16x8, u32x4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                                         __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)});
}
// 8 fp16 activations at byte `off` in natural order
__device__ __forceinline__ f16x8 xs_x8(__amdgpu_buffer_rsrc_t xr, uint32_t off) {
  return __builtin_bit_cast(f16x8, bld16(xr, off));
}

// The four words of a as floats.  Each element is copied to a scalar before the
// bit cast: a bit cast of a vector element expression itself has produced element 0.
__device__ __forceinline__ void xs_u4_to_f(u32x4 a, float* f) {
  const uint32_t t0 = a.x, t1 = a.y, t2 = a.z, t3 = a.w;
  f[0] = __builtin_bit_cast(float, t0);
  f[1] = __builtin_bit_cast(float, t1);
  f[2] = __builtin_bit_cast(float, t2);
  f[3] = __builtin_bit_cast(float, t3);
}

// 8 consecutive fp32 activations at byte `off`, reordered by ORD (index of the source
// element for each position)
template <int O0, int O1, int O2, int O3, int O4, int O5, int O6, int O7>
__device__ __forceinline__ void xs_x8_f32(__amdgpu_buffer_rsrc_t xr, uint32_t off, float (&v)[8]) {
  float f[8];
  xs_u4_to_f(bld16(xr, off), f);
  xs_u4_to_f(bld16(xr, off + 16u), f + 4);
  v[0] = f[O0]; v[1] = f[O1]; v[2] = f[O2]; v[3] = f[O3]; v[4] = f[O4]; v[5] = f[O5]; v[6] = f[O6]; v[7] = f[O7];
}
__device__ __forceinline__ f32x4 xs_mfma32(f16x8 a, u32x4 b, f32x4 d) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, __builtin_bit_cast(f16x8, b), d, 0, 0, 0);
}
constexpr f16x8 kXsOnes = {1, 1, 1, 1, 1, 1, 1, 1};

template <int I, int N, class Fn>
__device__ __forceinline__ void xs_static_for(Fn&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>());
    xs_static_for<I + 1, N>(f);
  }
}

// Dequant of two 4/6-bit quants held as fp16 denormals (q 2^-24, the halves of `a`):
// RN16(s * (q 2^-24) + c) for each half, with s = the weight scale times 2^24.  The
// compiler emits this as v_fma_mixlo/hi_f16 (fp32 fma of the converted half, one
// rounding to fp16), so each weight is the exact value rounded once.
__device__ __forceinline__ uint32_t xs_dq2(uint32_t a, float s, float c) {
  const f16x2 v = __builtin_bit_cast(f16x2, a);
  const f16x2 o = {(_Float16)__builtin_fmaf(s, (float)v.x, c), (_Float16)__builtin_fmaf(s, (float)v.y, c)};
  return __builtin_bit_cast(uint32_t, o);
}

// Q4_K: unit = one 144-byte super-block; one chain per 32-element sub-block J (one
// 16x16x32 MFMA).  The lane reads the 16-byte header and bytes 8kq .. 8kq+7 of each
// 32-byte quant pair p (low nibbles: sub-block 2p, high: 2p+1, as 1024 + 16q).
struct XsQ4K {
  static constexpr int NCH = 8;
  static constexpr bool WIDE = true;             // 16 slots per wave and 2 tiles fit
  struct Raw { u32x4 hd; uint2 q[4]; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 144u;
    r.hd = bld16(src.w, bo);
#pragma unroll
    for (int p = 0; p < 4; ++p)
      r.q[p] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(src.w, bo + 16u + 32u * p + 8u * kq, 0, 0));
  }
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8_perm4(xr, off + 2u * (uint32_t)(32 * S + 8 * kq));
  }
  __device__ static void xload32(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq, float (&v)[8]) {
    xs_x8_f32<0, 2, 1, 3, 4, 6, 5, 7>(xr, off + 4u * (uint32_t)(32 * S + 8 * kq), v);
  }
  template <int C>
  __device__ static f32x4 chain(const f16x8* xu, const Raw& r) {
    constexpr int p = C >> 1;
    constexpr uint32_t m = (C & 1) ? 0x00F000F0u : 0x000F000Fu;
    const uint32_t w0 = r.q[p].x, w1 = r.q[p].y;
    const u32x4 b = {(w0 & m) | kXsMagic, ((w0 >> 8) & m) | kXsMagic, (w1 & m) | kXsMagic, ((w1 >> 8) & m) | kXsMagic};
    return xs_mfma32(xu[C], b, f32x4{0.f, 0.f, 0.f, 0.f});
  }
  template <int C>
  __device__ static f32x4 xsum(const f16x8* xu) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(xu[C], kXsOnes, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  }
  template <int C>
  __device__ static void sc(const Raw& r, float& s, float& c) {
    uint32_t scl, mn;
    q4k_scale_min(r.hd.y, r.hd.z, r.hd.w, C, scl, mn);
    s = h2f(r.hd.x) * (float)scl * ((C & 1) ? 0.0625f : 1.f);
    c = -(h2f(r.hd.x >> 16) * (float)mn) - 1024.f * s;
  }
  // chain C with the weights dequantised to fp16 (d sc q - dmin m, rounded once),
  // accumulated into acc; nibbles masked in place (high ones as 16 q, scale / 16)
  template <int C>
  __device__ static void dq(const f16x8* xu, const Raw& r, f32x4& acc) {
    constexpr int p = C >> 1;
    constexpr uint32_t m = (C & 1) ? 0x00F000F0u : 0x000F000Fu;
    uint32_t scl, mn;
    q4k_scale_min(r.hd.y, r.hd.z, r.hd.w, C, scl, mn);
    const float s = h2f(r.hd.x) * (float)scl * ((C & 1) ? 1048576.f : 16777216.f);
    const float c = -(h2f(r.hd.x >> 16) * (float)mn);
    const uint32_t w0 = r.q[p].x, w1 = r.q[p].y;            // pairs in the xload order
    const u32x4 b = {xs_dq2(w0 & m, s, c), xs_dq2((w0 >> 8) & m, s, c), xs_dq2(w1 & m, s, c),
                     xs_dq2((w1 >> 8) & m, s, c)};
    acc = xs_mfma32(xu[C], b, acc);
  }
};

// MLX 4-bit affine, group size 32 << GSH: unit = 128 qweight bytes = 32 words of 8
// elements (element e of a word at bits 4e).  The lane reads LW = 1, 2 or 4
// consecutive words per load (LW = 2^min(GSH, 2)); load l of lane kq covers words
// 4 LW l + LW kq + h (h < LW), and MFMA J = LW l + h takes word slot h of load l, so
// the four lanes of one MFMA read four words of one group (a group is 4 << GSH
// words).  One chain per group of the unit (its MFMAs share the scale and bias).
// Scales and biases of the unit's groups: a row's groups are contiguous.
template <int GSH>
struct XsMLX {
  static constexpr int LW = GSH >= 2 ? 4 : 1 << GSH;    // words per lane load
  static constexpr int G = GSH >= 3 ? 1 : 8 >> GSH;     // groups per unit
  static constexpr int NW = G >= 2 ? G / 2 : 1;         // scale words per unit
  static constexpr int CH = 8 / G;                      // MFMAs per chain
  static constexpr int NCH = G;
  static constexpr bool WIDE = true;
  struct Raw { uint32_t q[8]; uint32_t sc[NW], bi[NW]; };
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
  // slot S = MFMA S: word 4 LW (S / LW) + LW kq + S % LW of the unit
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8_perm8(xr, off + 16u * (uint32_t)(4 * LW * (S / LW) + LW * kq + S % LW));
  }
  __device__ static void xload32(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq, float (&v)[8]) {
    xs_x8_f32<0, 4, 1, 5, 2, 6, 3, 7>(xr, off + 32u * (uint32_t)(4 * LW * (S / LW) + LW * kq + S % LW), v);
  }
  template <int C>
  __device__ static f32x4 chain(const f16x8* xu, const Raw& r) {
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const uint32_t w = r.q[C * CH + i];
      const u32x4 b = {(w & 0x000F000Fu) | kXsMagic, ((w >> 4) & 0x000F000Fu) | kXsMagic,
                       ((w >> 8) & 0x000F000Fu) | kXsMagic, ((w >> 12) & 0x000F000Fu) | kXsMagic};
      d = xs_mfma32(xu[C * CH + i], b, d);
    }
    return d;
  }
  template <int C>
  __device__ static f32x4 xsum(const f16x8* xu) {
    f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < CH; ++i) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(xu[C * CH + i], kXsOnes, d, 0, 0, 0);
    return d;
  }
  template <int C>
  __device__ static void sc(const Raw& r, float& s, float& c) {
    s = h2f(r.sc[C >> 1] >> (16 * (C & 1)));
    c = h2f(r.bi[C >> 1] >> (16 * (C & 1))) - 1024.f * s;
  }
};

// Q6_K: unit = one 210-byte super-block (2-byte aligned in the row).  One chain per
// 16-element scale group C (element 16 C + l, l < 16; group C = sub-block C / 2 of
// 32, half C % 2), one 16x16x16 MFMA: lane kq supplies elements 16 C + 4 kq .. + 3,
// as 1024 + (ql nibble | qh bits << 4) (the stored 6-bit value; q = that - 32).
// Element e = 128 h + 32 s + l: ql byte 64 h + 32 (s & 1) + l, nibble 4 (s >> 1);
// qh byte 128 + 32 h + l, bits 2 s; scale byte 192 + C (int8); d at byte 208.
// The lane's ql dwords m = 4 h + 2 (s & 1) + (l >= 16) and qh dwords m' = 2 h + (l >= 16)
// are read with 8-byte loads from the 4-byte aligned address below and realigned.
struct XsQ6K {
  static constexpr int NCH = 16;
  static constexpr bool WIDE = false;            // (a 16-slot wave or 2 tiles would spill)
  struct Raw { uint32_t ql[8], qh[4], scw[4], d; };
  __device__ static uint32_t word_a2(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const uint32_t sh = off & 2u;
    const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off - sh, 0, 0));
    return __builtin_amdgcn_alignbyte(v.y, v.x, sh);
  }
  __device__ static void load(const Src& src, uint32_t rw, uint32_t, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 210u;
#pragma unroll
    for (int m = 0; m < 8; ++m) r.ql[m] = word_a2(src.w, bo + 16u * m + 4u * kq);
#pragma unroll
    for (int m = 0; m < 4; ++m) r.qh[m] = word_a2(src.w, bo + 128u + 16u * m + 4u * kq);
    {
      const uint32_t so = bo + 192u, sh = so & 2u, base = so - sh;
      const u32x4 a = bld16(src.w, base);
      const uint32_t e = bld4(src.w, base + 16u);
      r.scw[0] = __builtin_amdgcn_alignbyte(a.y, a.x, sh);
      r.scw[1] = __builtin_amdgcn_alignbyte(a.z, a.y, sh);
      r.scw[2] = __builtin_amdgcn_alignbyte(a.w, a.z, sh);
      r.scw[3] = __builtin_amdgcn_alignbyte(e, a.w, sh);
    }
    r.d = bld2(src.w, bo + 208u);
  }
  // slot S holds elements 32 S + 4 kq .. + 3 (low 4 halves) and 32 S + 16 + 4 kq .. + 3
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    const uint32_t o = off + 2u * (uint32_t)(32 * S + 4 * kq);
    const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(xr, o, 0, 0));
    const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(xr, o + 32u, 0, 0));
    return __builtin_bit_cast(f16x8, u32x4{lo.x, lo.y, hi.x, hi.y});
  }
  __device__ static void xload32(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq, float (&v)[8]) {
    const uint32_t o = off + 4u * (uint32_t)(32 * S + 4 * kq);
    xs_u4_to_f(bld16(xr, o), v);
    xs_u4_to_f(bld16(xr, o + 64u), v + 4);
  }
  __device__ static f16x4 half4(const f16x8& v, int hi) {
    return hi ? __builtin_shufflevector(v, v, 4, 5, 6, 7) : __builtin_shufflevector(v, v, 0, 1, 2, 3);
  }
  template <int C>
  __device__ static f32x4 chain(const f16x8* xu, const Raw& r) {
    constexpr int S = C >> 1, g2 = C & 1, h = S >> 2, s = S & 3;
    const uint32_t ql = r.ql[4 * h + 2 * (s & 1) + g2], qh = r.qh[2 * h + g2];
    const uint32_t v = ((ql >> (4 * (s >> 1))) & 0x0F0F0F0Fu) | (((qh >> (2 * s)) & 0x03030303u) << 4);
    const uint2 b = {__builtin_amdgcn_perm(0u, v, 0x0c010c00u) | kXsMagic, __builtin_amdgcn_perm(0u, v, 0x0c030c02u) | kXsMagic};
    return __builtin_amdgcn_mfma_f32_16x16x16f16(half4(xu[S], g2), __builtin_bit_cast(f16x4, b),
                                                  f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  }
  template <int C>
  __device__ static f32x4 xsum(const f16x8* xu) {
    const f16x4 ones = {1, 1, 1, 1};
    return __builtin_amdgcn_mfma_f32_16x16x16f16(half4(xu[C >> 1], C & 1), ones, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
  }
  template <int C>
  __device__ static void sc(const Raw& r, float& s, float& c) {
    s = h2f(r.d) * (float)(int8_t)((r.scw[C >> 2] >> (8 * (C & 3))) & 0xFFu);
    c = -1056.f * s;                              // (q - 32) with q stored as 1024 + q
  }
};

// Q6_K with the weights dequantised to fp16 (d sc (q - 32), rounded once), read as
// wide contiguous runs.  Lane kq owns the 64 elements 128 h + 32 s + l with h = kq / 2
// and s in {kq % 2, kq % 2 + 2} (l < 32): their low bits are the 32 ql bytes at 32 kq
// (nibble s / 2), their high bits the 32 qh bytes at 128 + 32 h (bits 2 s), their
// scales bytes 192 + 8 h + 2 s + l / 16, and d the fp16 at 208.  The unit starts only
// 2-byte aligned, so each run is loaded from the 4-byte boundary below it (8 loads of
// 2-16 bytes per unit and lane) and realigned by `sh` bytes when used.  No load that
// carries needed bytes reaches past the block (a load that only partly fits the buffer
// reads as zero whole, which would lose data of the buffer's last block): d has a
// 2-byte load of its own.  Slot S holds elements l = 8 (S % 4) .. + 7 of
// s = kq % 2 + 2 (S / 4), in natural order.
struct XsQ6KW {
  static constexpr int NCH = 8;
  static constexpr bool WIDE = false;
  static constexpr int MPW = 8;                  // 24 raw words per unit and buffer
  struct Raw { uint32_t ql[9], qh[9], sc[3], d, sh; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 210u, sh = bo & 2u, base = bo - sh;
    const uint32_t h = (uint32_t)kq >> 1;
    const u32x4 a0 = bld16(src.w, base + 32u * kq), a1 = bld16(src.w, base + 32u * kq + 16u);
    const u32x4 b0 = bld16(src.w, base + 128u + 32u * h), b1 = bld16(src.w, base + 144u + 32u * h);
    // the scales' run as 8 + 4 bytes: the third word is needed only when sh = 2, and
    // then it lies inside the block (a load that only partly fits the buffer would
    // read as zero whole)
    const uint2 c0 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(src.w, base + 192u + 8u * h, 0, 0));
    r.ql[0] = a0.x; r.ql[1] = a0.y; r.ql[2] = a0.z; r.ql[3] = a0.w;
    r.ql[4] = a1.x; r.ql[5] = a1.y; r.ql[6] = a1.z; r.ql[7] = a1.w;
    r.ql[8] = bld4(src.w, base + 32u * kq + 32u);
    r.qh[0] = b0.x; r.qh[1] = b0.y; r.qh[2] = b0.z; r.qh[3] = b0.w;
    r.qh[4] = b1.x; r.qh[5] = b1.y; r.qh[6] = b1.z; r.qh[7] = b1.w;
    r.qh[8] = bld4(src.w, base + 160u + 32u * h);
    r.sc[0] = c0.x; r.sc[1] = c0.y; r.sc[2] = bld4(src.w, base + 200u + 8u * h);
    r.d = bld2(src.w, bo + 208u);
    r.sh = sh * 8u;                                // as a bit shift
  }
  __device__ static uint32_t al(uint32_t hi, uint32_t lo, uint32_t shb) {
    return __builtin_amdgcn_alignbit(hi, lo, shb);      // (hi:lo) >> shb, shb < 32
  }
  // slot S: elements 128 (kq / 2) + 32 (kq % 2 + 2 (S / 4)) + 8 (S % 4) .. + 7
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8(xr, off + 2u * (uint32_t)(128 * (kq >> 1) + 32 * ((kq & 1) + 2 * (S >> 2)) + 8 * (S & 3)));
  }
  __device__ static void xload32(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq, float (&v)[8]) {
    xs_x8_f32<0, 1, 2, 3, 4, 5, 6, 7>(xr, off + 4u * (uint32_t)(128 * (kq >> 1) + 32 * ((kq & 1) + 2 * (S >> 2)) + 8 * (S & 3)), v);
  }
  template <int C>
  __device__ static void dq(const f16x8* xu, const Raw& r, f32x4& acc) {
    constexpr int hi = C >> 2, l0 = 8 * (C & 3), wq = l0 / 4;
    const uint32_t shb = r.sh;
    // the lane's kq % 2 (not a template value): s = kq % 2 + 2 hi
    const uint32_t kq1 = (__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) >> 4) & 1u;
    const uint32_t qsh = 2u * kq1 + 4u * hi;
    // realigned scale words: bytes 8 h + 0..3 and + 4..7 of the scales; the slot's
    // scale is byte 2 (kq % 2) + (l0 >= 16) of word hi
    const uint32_t scw = hi ? al(r.sc[2], r.sc[1], shb) : al(r.sc[1], r.sc[0], shb);
    const int scb = __builtin_amdgcn_sbfe((int)scw, (int)(16u * kq1 + (l0 >= 16 ? 8u : 0u)), 8);
    const float sc = h2f(r.d) * (float)scb, sm = sc * 16777216.f, c = -32.f * sc;
    uint32_t b[4];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const uint32_t v = al(r.ql[wq + k + 1], r.ql[wq + k], shb), u = al(r.qh[wq + k + 1], r.qh[wq + k], shb);
      // u rotated right by qsh - 4: each byte's 2-bit field lands at its bits 4-5
      const uint32_t ur = __builtin_amdgcn_alignbit(u, u, (qsh + 28u) & 31u);
      const uint32_t q4 = bfi(0x30303030u, ur, (v >> (4 * hi)) & 0x0F0F0F0Fu);
      b[2 * k] = xs_dq2(__builtin_amdgcn_perm(0u, q4, 0x0c010c00u), sm, c);
      b[2 * k + 1] = xs_dq2(__builtin_amdgcn_perm(0u, q4, 0x0c030c02u), sm, c);
    }
    acc = xs_mfma32(xu[C], u32x4{b[0], b[1], b[2], b[3]}, acc);
  }
};

// GGUF wire Q5_0 / Q8_0 with the weights dequantised to fp16 (d (q - 16) / d q, rounded
// once).  Unit = 8 blocks of 32 (Q5_0 176 B, Q8_0 272 B: a 16-byte multiple, so with a
// 4-byte-aligned blob every unit starts 4-byte aligned); lane kq owns blocks 2 kq and
// 2 kq + 1, read with 16-byte loads from its 4-byte-aligned start and realigned in
// registers.  Slot S of lane kq holds the lane's elements 8 S .. 8 S + 7 (block S / 4,
// elements 8 (S % 4) .. + 7) in natural order, so the activations enter the MFMA as
// loaded (no reorder waits on their loads).
struct XsQ50 {
  static constexpr int NCH = 8;
  static constexpr bool WIDE = false;
  struct Raw { uint32_t w[11]; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 176u + 44u * (uint32_t)kq;
    const u32x4 a = bld16(src.w, bo), b = bld16(src.w, bo + 16u);
    const auto c = __builtin_amdgcn_raw_buffer_load_b96(src.w, bo + 32u, 0, 0);
    r.w[0] = a.x; r.w[1] = a.y; r.w[2] = a.z; r.w[3] = a.w;
    r.w[4] = b.x; r.w[5] = b.y; r.w[6] = b.z; r.w[7] = b.w;
    r.w[8] = c[0]; r.w[9] = c[1]; r.w[10] = c[2];
  }
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8(xr, off + 2u * (uint32_t)(64 * kq + 8 * S));
  }
  // block A at byte 0: d | qh at 2 | qs at 6; block B at byte 22: d | qh at 24 | qs at 28
  __device__ static uint32_t qs(const Raw& r, int blk, int i) {
    return blk ? r.w[7 + i] : __builtin_amdgcn_alignbyte(r.w[2 + i], r.w[1 + i], 2);
  }
  __device__ static uint32_t qh(const Raw& r, int blk) {
    return blk ? r.w[6] : __builtin_amdgcn_alignbyte(r.w[1], r.w[0], 2);
  }
  template <int C>
  __device__ static void dq(const f16x8* xu, const Raw& r, f32x4& acc) {
    constexpr int blk = C >> 2, j0 = 8 * (C & 3), nsh = 4 * ((C >> 1) & 1), wi = 2 * (C & 1);
    const float dd = h2f(blk ? r.w[5] >> 16 : r.w[0]), s = dd * 16777216.f, c = -16.f * dd;
    const uint32_t h = qh(r, blk);
    uint32_t b[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // elements (2p, 2p + 1): bytes 2 (p & 1) and + 1 of qs word wi + p / 2, their
      // nibble at nsh, qh bits j0 + 2p and + 1 moved to bits 4 and 20
      const uint32_t v = __builtin_amdgcn_perm(0u, qs(r, blk, wi + (p >> 1)), (p & 1) ? 0x0c030c02u : 0x0c010c00u);
      const uint32_t hb = (__builtin_amdgcn_ubfe(h, j0 + 2 * p, 2) * 0x00080010u) & 0x00100010u;
      b[p] = xs_dq2(((v >> nsh) & 0x000F000Fu) | hb, s, c);
    }
    acc = xs_mfma32(xu[C], u32x4{b[0], b[1], b[2], b[3]}, acc);
  }
};

struct XsQ80 {
  static constexpr int NCH = 8;
  static constexpr bool WIDE = false;
  struct Raw { uint32_t w[17]; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 272u + 68u * (uint32_t)kq;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 a = bld16(src.w, bo + 16u * i);
      r.w[4 * i] = a.x; r.w[4 * i + 1] = a.y; r.w[4 * i + 2] = a.z; r.w[4 * i + 3] = a.w;
    }
    r.w[16] = bld4(src.w, bo + 64u);
  }
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8(xr, off + 2u * (uint32_t)(64 * kq + 8 * S));
  }
  // block A at byte 0: d | qs at 2; block B at byte 34: d | qs at 36
  __device__ static uint32_t qs(const Raw& r, int blk, int i) {
    return blk ? r.w[9 + i] : __builtin_amdgcn_alignbyte(r.w[1 + i], r.w[i], 2);
  }
  template <int C>
  __device__ static void dq(const f16x8* xu, const Raw& r, f32x4& acc) {
    constexpr int blk = C >> 2, wi = 2 * (C & 3);
    const float dd = h2f(blk ? r.w[8] >> 16 : r.w[0]), s = dd * 16777216.f, c = -128.f * dd;
    uint32_t b[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // int8 q as the byte q + 128 (fp16 denormal (q + 128) 2^-24): elements 2p, 2p + 1
      const uint32_t v = __builtin_amdgcn_perm(0u, qs(r, blk, wi + (p >> 1)), (p & 1) ? 0x0c030c02u : 0x0c010c00u);
      b[p] = xs_dq2(v ^ 0x00800080u, s, c);
    }
    acc = xs_mfma32(xu[C], u32x4{b[0], b[1], b[2], b[3]}, acc);
  }
};

// Q8_0 in the split layout (int8 quants [N, K], fp16 scales [N, K/32]): lane kq of a
// 256-element unit takes its 64 contiguous quants (four aligned 16-byte loads) and its
// two blocks' scales (one dword); the chains and the dequant are XsQ80's.
struct XsQ80S {
  static constexpr int NCH = 8;
  static constexpr bool WIDE = false;
  struct Raw { uint32_t w[16]; uint32_t d; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t rs, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 256u + 64u * (uint32_t)kq;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 a = bld16(src.w, bo + 16u * i);
      r.w[4 * i] = a.x; r.w[4 * i + 1] = a.y; r.w[4 * i + 2] = a.z; r.w[4 * i + 3] = a.w;
    }
    r.d = bld4(src.s, rs + (uint32_t)unit * 16u + 4u * (uint32_t)kq);
  }
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8(xr, off + 2u * (uint32_t)(64 * kq + 8 * S));
  }
  template <int C>
  __device__ static void dq(const f16x8* xu, const Raw& r, f32x4& acc) {
    constexpr int blk = C >> 2, wi = 2 * (C & 3);
    const float dd = h2f(blk ? r.d >> 16 : r.d), s = dd * 16777216.f, c = -128.f * dd;
    uint32_t b[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // int8 q as the byte q + 128 (fp16 denormal (q + 128) 2^-24): elements 2p, 2p + 1
      const uint32_t v = __builtin_amdgcn_perm(0u, r.w[8 * blk + wi + (p >> 1)], (p & 1) ? 0x0c030c02u : 0x0c010c00u);
      b[p] = xs_dq2(v ^ 0x00800080u, s, c);
    }
    acc = xs_mfma32(xu[C], u32x4{b[0], b[1], b[2], b[3]}, acc);
  }
};

// Q5_0 in the split layout (qweight u8[N, K/2] K-sequential nibbles, qhigh u8[N, K/2]
// with element k's 5th bit at bit 0 and element k + 1's at bit 4 of byte k / 2, fp16
// scales [N, K/32]): lane kq of a 256-element unit takes its 64 contiguous elements
// (two 16-byte loads each of qweight and qhigh) and its two blocks' scales (one
// dword).  Chain C is slot C: elements 64 kq + 8 C .. + 7 in natural order, from
// word C of each array; the even elements' 5-bit values are formed in the bytes of
// one word, the odd ones' in another, and one byte permute per pair interleaves
// them into the fp16 halves (denormal integers), dequantised as d (u - 16).
struct XsQ50S {
  static constexpr int NCH = 8;
  static constexpr bool WIDE = false;
  struct Raw { uint32_t q[8], h[8]; uint32_t d; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t rs, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 128u + 32u * (uint32_t)kq;
    const u32x4 q0 = bld16(src.w, bo), q1 = bld16(src.w, bo + 16u);
    const u32x4 h0 = bld16(src.aux, bo), h1 = bld16(src.aux, bo + 16u);
    r.q[0] = q0.x; r.q[1] = q0.y; r.q[2] = q0.z; r.q[3] = q0.w;
    r.q[4] = q1.x; r.q[5] = q1.y; r.q[6] = q1.z; r.q[7] = q1.w;
    r.h[0] = h0.x; r.h[1] = h0.y; r.h[2] = h0.z; r.h[3] = h0.w;
    r.h[4] = h1.x; r.h[5] = h1.y; r.h[6] = h1.z; r.h[7] = h1.w;
    r.d = bld4(src.s, rs + (uint32_t)unit * 16u + 4u * (uint32_t)kq);
  }
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8(xr, off + 2u * (uint32_t)(64 * kq + 8 * S));
  }
  template <int C>
  __device__ static void dq(const f16x8* xu, const Raw& r, f32x4& acc) {
    constexpr int blk = C >> 2;
    const float dd = h2f(blk ? r.d >> 16 : r.d), s = dd * 16777216.f, c = -16.f * dd;
    const uint32_t q = r.q[C], h = r.h[C];
    // byte j: even element 2j (low nibble, 5th bit at bit 0), odd element 2j + 1 (high
    // nibble, 5th bit at bit 4)
    const uint32_t ev = bfi(0x0F0F0F0Fu, q, (h & 0x01010101u) << 4);
    const uint32_t od = bfi(0x0F0F0F0Fu, q >> 4, h & 0x10101010u);
    uint32_t b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)   // halves (element 2j, element 2j + 1)
      b[j] = xs_dq2(__builtin_amdgcn_perm(od, ev, 0x0c000c00u | (uint32_t)j | ((uint32_t)(4 + j) << 16)), s, c);
    acc = xs_mfma32(xu[C], u32x4{b[0], b[1], b[2], b[3]}, acc);
  }
};

// MLX 4-bit affine with the weights dequantised to fp16 (s q + b, rounded once), any
// group size 32 << GSH: every lane reads two 16-byte runs of four words (words 4 kq
// .. + 3 and 16 + 4 kq .. + 3 of the unit; MFMA S takes word 16 (S / 4) + 4 kq + S % 4),
// whatever the group size, since one MFMA may now span scale groups; each lane
// decodes the scale / bias of its two groups only.  Half the load instructions of the
// exact-integer MLX provider at group size 32 / 64.
template <int GSH>
struct XsMLXD {
  static constexpr int G = GSH >= 3 ? 1 : 8 >> GSH;     // groups per unit
  static constexpr int NW = G >= 2 ? G / 2 : 1;         // scale words per unit
  static constexpr int NCH = 8;
  static constexpr bool WIDE = true;
  static constexpr bool DQ = true;
  struct Raw { u32x4 q0, q1; uint32_t sc[NW], bi[NW]; };
  __device__ static void load(const Src& src, uint32_t rw, uint32_t rs, int unit, int kq, Raw& r) {
    const uint32_t bo = rw + (uint32_t)unit * 128u + 16u * kq;
    r.q0 = bld16(src.w, bo);
    r.q1 = bld16(src.w, bo + 64u);
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
  __device__ static uint32_t word(int S, int kq) { return (uint32_t)(16 * (S >> 2) + 4 * kq + (S & 3)); }
  __device__ static f16x8 xload(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq) {
    return xs_x8_perm8(xr, off + 16u * word(S, kq));
  }
  __device__ static void xload32(__amdgpu_buffer_rsrc_t xr, uint32_t off, int S, int kq, float (&v)[8]) {
    xs_x8_f32<0, 4, 1, 5, 2, 6, 3, 7>(xr, off + 32u * word(S, kq), v);
  }
  // scale and bias halves (as dwords shifted into the low half) of the lane's group for
  // words 16 h + 4 kq + (0..3): group (16 h + 4 kq) >> (2 + GSH)
  __device__ static void group(const Raw& r, int h, int kq, uint32_t& sc, uint32_t& bi) {
    if constexpr (GSH == 0) {                      // group 4 h + kq: word 2 h + kq / 2, half kq % 2
      const int wd = kq >> 1, sh = 16 * (kq & 1);
      sc = (wd ? r.sc[2 * h + 1] : r.sc[2 * h]) >> sh;
      bi = (wd ? r.bi[2 * h + 1] : r.bi[2 * h]) >> sh;
    } else if constexpr (GSH == 1) {               // group 2 h + kq / 2: word h, half kq / 2
      const int sh = 16 * (kq >> 1);
      sc = r.sc[h] >> sh;
      bi = r.bi[h] >> sh;
    } else if constexpr (GSH == 2) {               // group h
      sc = r.sc[0] >> (16 * h);
      bi = r.bi[0] >> (16 * h);
    } else {
      sc = r.sc[0];
      bi = r.bi[0];
    }
  }
  __device__ static void dq_unit(const f16x8* xu, const Raw& r, f32x4& acc) {
    const int kq = (int)(threadIdx.x >> 4) & 3;
    const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      uint32_t scw, biw;
      group(r, h, kq, scw, biw);
      const float sg = h2f(scw), c = h2f(biw);
      const float s0 = sg * 16777216.f, s1 = sg * 1048576.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = q[4 * h + i], w8 = w >> 8;
        // (e0,e4) (16e1,16e5) (e2,e6) (16e3,16e7): the xload order
        const u32x4 b = {xs_dq2(w & 0x000F000Fu, s0, c), xs_dq2(w & 0x00F000F0u, s1, c), xs_dq2(w8 & 0x000F000Fu, s0, c),
                         xs_dq2(w8 & 0x00F000F0u, s1, c)};
        acc = xs_mfma32(xu[4 * h + i], b, acc);
      }
    }
  }
};

// The same providers with the weights dequantised to fp16 before the MFMA (one
// rounding per weight) and accumulated across chains in the MFMA: no per-chain fp32
// fold and no activation sums.
template <class P>
struct XsDQ : P {
  static constexpr bool DQ = true;
  __device__ static void dq_unit(const f16x8* xu, const typename P::Raw& r, f32x4& acc) {
    xs_static_for<0, P::NCH>([&](auto cc) { P::template dq<decltype(cc)::value>(xu, r, acc); });
  }
};
// Waves per workgroup of the multi-pass kernel (MP): 16 by default (activations of a
// pass loaded after the previous pass's MFMAs, 128 VGPRs), 8 for providers whose raw
// bytes need the 256 VGPRs of an 8-wave workgroup (activations double-buffered too).
template <class P, class = void>
struct XsMPW : std::integral_constant<int, 16> {};
template <class P>
struct XsMPW<P, std::void_t<decltype(P::MPW)>> : std::integral_constant<int, P::MPW> {};
template <class P, class = void>
struct XsIsDQ : std::false_type {};
template <class P>
struct XsIsDQ<P, std::void_t<decltype(P::DQ)>> : std::bool_constant<P::DQ> {};

// ---------------------------------------------------------------- jobs
// MODE 0: dense y[t, n] = x[t] . W[n] for t < M (x [M, xld] fp16, y fp16 or fp32).
// MODE 1: routed gate/up.  Workgroup row y = column tile (expert e, sorted routes
//         p0 .. p0+cnt); token slot t gathers x[token t of the record]; weight rows
//         e*2N + n (gate) and e*2N + N + n (up); h[p0+t, n] = silu(gate) * up (fp32).
// MODE 2: routed down: x = h[p0+t] (fp32); weight rows e*N + n; part[p0+t, n] (fp32).
// MODE 3: dense gated pair y[t, n] = act(x[t] . G[n]) * (x[t] . U[n]) for t < M, with
//         G = a and U = a2 (y fp16 or fp32).
//         Each token's activations enter the MFMA as fp16 after a power-of-two
//         scaling that puts the token's largest |h| in [2^14, 2^15) (fp16 range,
//         11-bit precision whatever the magnitude); the result is scaled back.
struct XsJob {
  QArgs a;                 // whole matrix (all experts for MODE 1/2; the gate for MODE 3)
  QArgs a2;                // MODE 3: the up matrix (same format and shape as a)
  int act;                 // MODE 3: 0 silu, 1 gelu (tanh form)
  uint32_t sb;             // bytes per row of scales / biases (MLX), else 0
  const void* x;           // fp16 (MODE 0/1) or fp32 (MODE 2) activations
  uint32_t xbytes;         // bytes of x readable (bounds of the activation buffer)
  int xld;                 // elements per activation row
  int M;                   // MODE 0: activation rows; MODE 1/2: bound on routes per tile
  int N;                   // output rows (per matrix for MODE 1)
  void* y;                 // MODE 0 output [M, N]
  int y_f32;
  const int32_t* tiles;    // MODE 1/2: column tile records, kTileInts ints each
  const int32_t* ntiles;   // number of valid records
  float* h;                // MODE 1 output
  float* part;             // MODE 2 output
  int W;                   // waves per workgroup (set by the launcher)
  int kp;                  // K passes (multi-pass kernel; set by the launcher)
  int ku_split;            // MODE 0: 256-element units per K split (grid.y = split s
                           // takes units [s ku_split, (s + 1) ku_split) and writes fp32
                           // partials to y + s M N); 0: no split
};

// a * b rounded to fp32.  The empty asm (no instruction) pins the fp32 value: without
// it the compiler fuses the product with a following fp16 conversion (v_fma_mix,
// one rounding), which can differ from rounding the fp32 output.
__device__ __forceinline__ float xs_f32_product(float a, float b) {
  float p = a * b;
  asm volatile("" : "+v"(p));
  return p;
}

// Gate activations of the fused gated pair: silu(v) = v / (1 + e^-v); gelu in the
// tanh form 0.5 v (1 + tanh(clamp(sqrt(2/pi) (v + 0.044715 v^3), -10, 10))).
__device__ __forceinline__ float xs_act(int act, float v) {
  if (act == 0) return v * __builtin_amdgcn_rcpf(1.f + __expf(-v));
  const float u = fminf(fmaxf(0.7978845608028654f * (v + 0.044715f * v * v * v), -10.f), 10.f);
  return 0.5f * v * (1.f + tanhf(u));
}


// NS: sub-blocks per wave (8 or 16); TT: token slots folded per lane (lanes 16 kq
// hold tokens 4 kq .. 4 kq + 3, so at most TT <= 4 active rows need only the first
// TT); RT: 16-row tiles per reduction.  MP (MODE 0, RT = 1, dequantising providers,
// at most XsMPW waves): K longer than the W waves' slots is covered in j.kp passes,
// pass p giving wave w the units (p W + w) UPW ..; the tile's accumulators carry over
// the passes, and the weights of pass p + 1 are requested before pass p is computed.
// Otherwise the tile loop is
// software-pipelined over two register sets: the weights of the workgroup's next
// RT tiles are requested before the current ones are used (PIPE), and the first
// tiles' weights are requested before the activations are waited for.  Rows past the
// matrix, tiles past the end and activations past the buffers read as zero (buffer
// bounds, no memory traffic); outputs past the valid rows and tokens are not
// stored.  Dynamic LDS: Xs[W][NS/8][NCH][16] + red[W][RT][64][4 NM] (+ tmx[W][16]
// + tsc[16] for MODE 2) floats.
template <class P, int MODE, int NS, int TT, int RT, bool PIPE, class YT, bool MP = false>
__device__ __forceinline__ void xs_body(const XsJob& j) {
  static_assert(!MP || (MODE == 0 && RT == 1 && !PIPE && XsIsDQ<P>::value), "multi-pass: dense, one tile, dequantising");
  constexpr int NM = (MODE == 1 || MODE == 3) ? 2 : 1;   // weight matrices per output
  constexpr int UPW = NS / 8;                    // units per wave
  constexpr int NCH = P::NCH;                    // chains per unit
  using Raw = typename P::Raw;
  extern __shared__ __attribute__((aligned(16))) float xs_smem[];
  const int K = j.a.K, KU = K >> 8;
  // the wave count comes from the arguments (scalar loads), not from blockDim: that
  // is read with a vector load, and one issued after the weight prefetch makes every
  // later wait drain the prefetch too
  const int W = j.W, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  float* Xs = xs_smem;                                   // [W][UPW][NCH][16]
  float* red = xs_smem + W * UPW * NCH * 16;             // [W][RT][64][4 NM]
  float* tmx = red + W * RT * 64 * 4 * NM;               // [W][16] token |x| maxima (MODE 2)
  float* tsc = tmx + W * 16;                             // [16] token scales (MODE 2)
  const int n16 = lane & 15, kq = lane >> 4;
  // this workgroup's units [ubase, uend): all of K, or its K split (MODE 0)
  int ubase = 0, uend = KU;
  int64_t yoff = 0;                                      // its output slice (K split: partials)
  if constexpr (MODE == 0) {
    if (j.ku_split > 0) {
      ubase = (int)blockIdx.y * j.ku_split;
      uend = KU - ubase < j.ku_split ? KU : ubase + j.ku_split;
      yoff = (int64_t)blockIdx.y * j.M * j.N;
    }
  }
  int u0 = ubase + wave * UPW;                           // first unit of this wave (this pass)
  int nu = uend - u0 < UPW ? uend - u0 : UPW;            // units present (uniform; <= 0: none)
  auto set_pass = [&](int p) {
    u0 = ubase + (p * W + wave) * UPW;
    nu = uend - u0 < UPW ? uend - u0 : UPW;
  };

  int cnt = j.M, p0 = 0, tok = 0;
  int64_t row0 = 0;                                      // first weight row of the block
  if constexpr (MODE == 1 || MODE == 2) {
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
  // one buffer view per weight matrix, N rows each (rows past N read zero)
  auto rows_from = [&](const QArgs& q, int64_t r0) {
    QArgs o = q;
    o.w += r0 * q.rb;
    if (o.s) o.s += r0 * (j.sb / 2);
    if (o.b) o.b += r0 * (j.sb / 2);
    return Src(o, (uint32_t)j.N * (uint32_t)q.rb, (uint32_t)j.N * j.sb);
  };
  Src src[NM];
  src[0] = rows_from(j.a, row0);
  if constexpr (MODE == 1) src[1] = rows_from(j.a, row0 + j.N);   // up rows follow the gate rows
  if constexpr (MODE == 3) src[1] = rows_from(j.a2, 0);
  const uint32_t rb = (uint32_t)j.a.rb;
  const int ntiles16 = (j.N + 15) >> 4;
  const int stride = (int)gridDim.x * RT;

  // request the weights of tiles t .. t+RT-1 (tiles past the end: out of bounds)
  auto load_tiles = [&](Raw (&raw)[RT][NM][UPW], int t) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const bool in = t + r < ntiles16;
      const uint32_t n = (uint32_t)((t + r) * 16 + n16);
      const uint32_t rw = in ? n * rb : 0x80000000u, rs = in ? n * j.sb : 0x80000000u;
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) {
#pragma unroll
        for (int u = 0; u < UPW; ++u) {
          const bool has = u < nu;                       // units past K: no traffic
          P::load(src[mi], has ? rw : 0x80000000u, has ? rs : 0x80000000u, u0 + u, kq, raw[r][mi][u]);
        }
      }
    }
  };

  // A operands: token slot n16, slots 8 u .. 8 u + 7 of unit u0 + u (provider order)
  f16x8 xa[NS];
  constexpr uint32_t XB = MODE == 2 ? 4u : 2u;           // bytes per activation
  auto load_x_to = [&](f16x8 (&xa)[NS]) {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc((void*)j.x, (short)0, (int)j.xbytes, ALLOY_RSRC_DW3);
    uint32_t xrow = 0x80000000u;                         // past the buffer: zeros
    if (n16 < cnt) {
      int64_t r = n16;
      if constexpr (MODE == 1) r = tok;
      else if constexpr (MODE == 2) r = p0 + n16;
      xrow = (uint32_t)(r * j.xld) * XB;
    }
    if constexpr (MODE != 2) {
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint32_t off = (s >> 3) < nu ? xrow + 512u * (uint32_t)(u0 + (s >> 3)) : 0x80000000u;
        xa[s] = P::xload(xr, off, s & 7, kq);
      }
    } else {
      float v[NS][8];
      float m = 0.f;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const uint32_t off = (s >> 3) < nu ? xrow + 1024u * (uint32_t)(u0 + (s >> 3)) : 0x80000000u;
        P::xload32(xr, off, s & 7, kq, v[s]);
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[s][i]));
      }
      // the token's largest |h| over the workgroup (lanes n16 + 16 kq, then the waves)
      m = fmaxf(m, __shfl_xor(m, 16, 64));
      m = fmaxf(m, __shfl_xor(m, 32, 64));
      if (kq == 0) tmx[wave * 16 + n16] = m;
      __syncthreads();
      float tm = 0.f;
      for (int w = 0; w < W; ++w) tm = fmaxf(tm, tmx[w * 16 + n16]);
      int ex = 0;
      if (tm > 0.f && tm <= 3.0e38f) (void)frexpf(tm, &ex);     // tm = f 2^ex, f in [0.5, 1)
      const int sh = tm > 0.f && tm <= 3.0e38f ? ex - 15 : 0;   // tm 2^-sh in [2^14, 2^15)
      const float down = ldexpf(1.f, -sh);
      if (wave == 0 && kq == 0) tsc[n16] = ldexpf(1.f, sh);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        f16x8 a;
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = (f16)(v[s][i] * down);
        xa[s] = a;
      }
    }
  };

  auto load_x = [&]() { load_x_to(xa); };

  // fold tile r of `raw` into acc (TTR token slots per lane)
  auto accumulate = [&](const Raw (&raw)[RT][NM][UPW], int r, f32x4 (&acc)[NM], auto ttc) {
    constexpr int TTR = decltype(ttc)::value;
    {
#pragma unroll
      for (int u = 0; u < UPW; ++u) {
        if (u >= nu) break;                      // uniform; keeps xa[] statically indexed
        if constexpr (XsIsDQ<P>::value) {
#pragma unroll
          for (int mi = 0; mi < NM; ++mi) P::dq_unit(&xa[8 * u], raw[r][mi][u], acc[mi]);
          continue;
        }
        xs_static_for<0, NCH>([&](auto cc) {
          constexpr int C = decltype(cc)::value;
          if constexpr (XsIsDQ<P>::value) {
          } else {
            const f32x4 xsum = *(const f32x4*)&Xs[((wave * UPW + u) * NCH + C) * 16 + 4 * kq];
#pragma unroll
            for (int mi = 0; mi < NM; ++mi) {
              const f32x4 d = P::template chain<C>(&xa[8 * u], raw[r][mi][u]);
              float sc, off;
              P::template sc<C>(raw[r][mi][u], sc, off);
#pragma unroll
              for (int tt = 0; tt < TTR; ++tt) {
                const float dv = d[tt];
                acc[mi][tt] += sc * dv + off * xsum[tt];
              }
            }
          }
        });
      }
    }
  };
  // reduce the accumulators of tiles t .. t+RT-1 over the waves, store
  auto finish = [&](const f32x4 (&acc)[RT][NM], int t, auto ttc) {
    constexpr int TTR = decltype(ttc)::value;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int mi = 0; mi < NM; ++mi)
        *(f32x4*)&red[((wave * RT + r) * 64 + lane) * (4 * NM) + 4 * mi] = acc[r][mi];
    // LDS-only barriers: a __syncthreads would also wait for the next tiles' weights
    // (its fence drains every outstanding load), serialising the prefetch
    lds_barrier();
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
        ((YT*)j.y)[yoff + (int64_t)tk * j.N + n] = (YT)v0;
      } else if constexpr (MODE == 3) {
        ((YT*)j.y)[(int64_t)tk * j.N + n] = (YT)xs_f32_product(xs_act(j.act, v0), v1);
      } else if constexpr (MODE == 1) {
        j.h[(int64_t)(p0 + tk) * j.N + n] = v0 * __builtin_amdgcn_rcpf(1.f + __expf(-v0)) * v1;
      } else {
        j.part[(int64_t)(p0 + tk) * j.N + n] = v0 * tsc[tk];
      }
    }
    lds_barrier();                                // red[] is reused by the next tiles
  };
  auto compute_tiles = [&](const Raw (&raw)[RT][NM][UPW], int t, auto ttc) {
    f32x4 acc[RT][NM];
#pragma unroll
    for (int r = 0; r < RT; ++r) {
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) acc[r][mi] = f32x4{0.f, 0.f, 0.f, 0.f};
      accumulate(raw, r, acc[r], ttc);
    }
    finish(acc, t, ttc);
  };

  Raw ra[RT][NM][UPW];
  int t = blockIdx.x * RT;
  if constexpr (MP) {
    // every pass computes all of its units: units past K were loaded as zeros (weights
    // and activations), which adds nothing, and there is no branch between a load and
    // its use that would make the compiler wait for the newer prefetch too.  Weights
    // alternate between ra and rc, one pass ahead; with 8 waves the activations too
    // (xa / xb), with 16 they are loaded after the previous pass's MFMAs.
    // Scheduling barriers keep each prefetch issued ahead of the MFMAs of the pass
    // before it (the waits then count only the older loads); passes past the last load
    // out of bounds (no traffic).
    const int KP = j.kp;
    const std::integral_constant<int, TT> ttc;
    constexpr bool X2 = XsMPW<P>::value <= 8;
    auto fold = [&](const Raw (&raw)[RT][NM][UPW], const f16x8 (&xv)[NS], f32x4 (&acc)[NM]) {
#pragma unroll
      for (int u = 0; u < UPW; ++u)
#pragma unroll
        for (int mi = 0; mi < NM; ++mi) P::dq_unit(&xv[8 * u], raw[0][mi][u], acc[mi]);
    };
    Raw rc[1][NM][UPW];
    f16x8 xb[X2 ? NS : 1];
    for (; t < ntiles16; t += stride) {          // uniform
      f32x4 acc[1][NM];
#pragma unroll
      for (int mi = 0; mi < NM; ++mi) acc[0][mi] = f32x4{0.f, 0.f, 0.f, 0.f};
      set_pass(0);
      load_tiles(ra, t);
      load_x_to(xa);
      if constexpr (X2) {
        set_pass(1);
        load_tiles(rc, t);
        load_x_to(xb);
        for (int p = 0; p < KP; p += 2) {        // passes in pairs: (ra, xa) even, (rc, xb) odd
          __builtin_amdgcn_sched_barrier(0);
          fold(ra, xa, acc[0]);
          set_pass(p + 2);
          load_tiles(ra, t);
          load_x_to(xa);
          __builtin_amdgcn_sched_barrier(0);
          fold(rc, xb, acc[0]);
          set_pass(p + 3);
          load_tiles(rc, t);
          load_x_to(xb);
        }
      } else {
        for (int p = 0; p < KP; p += 2) {        // passes in pairs: ra even, rc odd
          set_pass(p + 1);
          load_tiles(rc, t);
          __builtin_amdgcn_sched_barrier(0);
          fold(ra, xa, acc[0]);
          load_x_to(xa);
          set_pass(p + 2);
          load_tiles(ra, t);
          __builtin_amdgcn_sched_barrier(0);
          fold(rc, xa, acc[0]);
          load_x_to(xa);
        }
      }
      finish(acc, t, ttc);
    }
    return;
  }
  if constexpr (XsIsDQ<P>::value) {
    // weights first: the activations' reorder waits for their loads, which then
    // overlap the weights' instead of preceding them
    load_tiles(ra, t);
    load_x();
  } else {
    load_x();                                    // x first: its sums overlap the weight loads
    load_tiles(ra, t);
  }
  // X per chain: tokens 4kq .. 4kq+3 in lane 16 kq
  if constexpr (!XsIsDQ<P>::value) {
#pragma unroll
    for (int u = 0; u < UPW; ++u) {
      xs_static_for<0, NCH>([&](auto cc) {
        constexpr int C = decltype(cc)::value;
        const f32x4 X = P::template xsum<C>(&xa[8 * u]);
        if (n16 == 0) *(f32x4*)&Xs[((wave * UPW + u) * NCH + C) * 16 + 4 * kq] = X;
      });
    }
    __syncthreads();
  }
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

template <class P, int MODE, int NS, int TT, int RT, bool PIPE, class YT, bool MP = false>
__global__ __launch_bounds__(MP ? 64 * XsMPW<P>::value : 1024) void k_gemv_xs(XsJob j) {
  xs_body<P, MODE, NS, TT, RT, PIPE, YT, MP>(j);
}

// MODE 0 with the job's fields as scalar arguments, those the first loads need first:
// the dispatch preloads the leading ones into SGPRs, where a structure argument is
// read from memory before any load can be addressed.
template <class P, int NS, int TT, int RT, bool PIPE, class YT, bool MP = false>
__global__ __launch_bounds__(MP ? 64 * XsMPW<P>::value : 1024) void k_gemv_xs0(
    const uint8_t* w, int64_t rb, int K, const void* x, int W, int N, int M, int kp, int ku_split, uint32_t xbytes,
    int xld, void* y, const uint16_t* s, const uint16_t* b, uint32_t sb, int gs, const uint8_t* aux) {
  XsJob j{};
  j.a = QArgs{w, aux, s, b, rb, gs, K};
  j.x = x;
  j.xbytes = xbytes;
  j.xld = xld;
  j.M = M;
  j.N = N;
  j.y = y;
  j.sb = sb;
  j.W = W;
  j.kp = kp;
  j.ku_split = ku_split;
  xs_body<P, 0, NS, TT, RT, PIPE, YT, MP>(j);
}

// Host launcher.  hipErrorNotSupported when the shape does not fit the kernel
// (K not a multiple of 256, over 8192 except for the multi-pass dense kernel of the
// dequantising providers, offsets of 2 GiB or more): the caller then
// uses another kernel.  MODE 0: one 16-row tile (rt = 1) or two (rt = 2) per
// workgroup while the tiles fit the resident workgroups, else as many workgroups as
// are resident (or `cap`), each looping over tiles with the next tiles' weights in
// flight.  MODE 1/2: grid.y = `tiles_y` column tiles and grid.x = `cap` groups of
// output tiles per column tile (0: chosen here).
template <class P, int MODE>
hipError_t launch_xs(const XsJob& j, int64_t tiles_y, int64_t cap, int rt, hipStream_t st) {
  constexpr int NM = (MODE == 1 || MODE == 3) ? 2 : 1;
  constexpr bool DENSE = MODE == 0 || MODE == 3;
  const int K = j.a.K;
  if (K <= 0 || K % 256 || j.M > 16 || j.N <= 0) return hipErrorNotSupported;
  // K split (MODE 0): the plan below is that of one split's K
  const int KU = K / 256;
  const int ksplit = MODE == 0 && j.ku_split > 0 && j.ku_split < KU ? j.ku_split : 0;
  const int splits = ksplit ? (KU + ksplit - 1) / ksplit : 1;
  const uint64_t rows = (uint64_t)j.N + 16u;
  if (rows * (uint64_t)j.a.rb >= (1ull << 31) || rows * j.sb >= (1ull << 31) || j.xbytes >= (1u << 31))
    return hipErrorNotSupported;
  const int KS = (ksplit ? ksplit * 256 : K) / 32;
  int ns = KS <= 8 * 16 ? 8 : KS <= 16 * 16 ? 16 : 0;   // at most 16 waves
  int kp = 1;
  if (ns != 8 && MODE == 0 && XsIsDQ<P>::value && !P::WIDE) {
    constexpr int mw = XsMPW<P>::value;          // multi-pass: 8 slots per wave, <= mw waves
    ns = 8;
    kp = (KS + 8 * mw - 1) / (8 * mw);
  }
  if (!ns || ((NM == 2 || !P::WIDE) && ns == 16)) return hipErrorNotSupported;   // (registers)
  if (!DENSE && tiles_y > 65535) return hipErrorNotSupported;
  if (!DENSE && tiles_y <= 0) return hipSuccess;
  const int W = (KS + ns * kp - 1) / (ns * kp);
  const int64_t tiles = (j.N + 15) / 16;
  // 16 sub-blocks per wave leave registers for one tile in flight only
  rt = (ns == 16 || MODE != 0 || rt < 2 || !P::WIDE) ? 1 : 2;   // (two tiles: MODE 0 only)
  const int64_t groups = (tiles + rt - 1) / rt;
  const size_t lds = (size_t)W * (ns / 8) * P::NCH * 16 * 4 + (size_t)W * rt * 64 * 4 * NM * 4 +
                     (MODE == 2 ? (size_t)(W * 16 + 16) * 4 : 0);
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
      int64_t c = cap > 0 ? cap : (int64_t)resident_per_cu((const void*)kern, 64 * W, lds) * cu_count();
      c = c / splits > 0 ? c / splits : 1;              // the K splits share the resident slots
      gx = groups < c ? groups : c;
    }
    const dim3 grid((unsigned)gx, DENSE ? (unsigned)splits : (unsigned)tiles_y), block((unsigned)(64 * W));
    XsJob jw = j;
    jw.W = W;
    jw.kp = kp;
    jw.ku_split = ksplit;
    if constexpr (MODE == 0)
      hipLaunchKernelGGL(kern, grid, block, lds, st, jw.a.w, jw.a.rb, jw.a.K, jw.x, jw.W, jw.N, jw.M, jw.kp,
                         jw.ku_split, jw.xbytes, jw.xld, jw.y, jw.a.s, jw.a.b, jw.sb, jw.a.gs, jw.a.aux);
    else
      hipLaunchKernelGGL(kern, grid, block, lds, st, jw);
    return hipGetLastError();
  };
  // whether the tiles outnumber the resident workgroups of the one-pass kernel
  auto many = [&](auto kern) -> bool {
    const int64_t c = cap > 0 ? cap : (int64_t)resident_per_cu((const void*)kern, 64 * W, lds) * cu_count();
    return groups * splits > c;
  };
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I4 = std::integral_constant<int, 4>;
  if constexpr (MODE == 0) {
    auto pick = [&](auto ttc, auto yt) -> hipError_t {
      constexpr int TT = decltype(ttc)::value;
      using YT = decltype(yt);
      if constexpr (XsIsDQ<P>::value && !P::WIDE) {
        if (kp > 1) return go(k_gemv_xs0<P, 8, TT, 1, false, YT, true>, false);
      }
      if constexpr (P::WIDE) {
        if (ns == 16) return go(k_gemv_xs0<P, 16, TT, 1, false, YT>, false);
        if (rt == 2) return go(k_gemv_xs0<P, 8, TT, 2, true, YT>, true);
      }
      if (many(k_gemv_xs0<P, 8, TT, 1, false, YT>)) return go(k_gemv_xs0<P, 8, TT, 1, true, YT>, true);
      return go(k_gemv_xs0<P, 8, TT, 1, false, YT>, false);
    };
    if (j.y_f32) return tt == 1 ? pick(I1(), 0.f) : tt == 2 ? pick(I2(), 0.f) : pick(I4(), 0.f);
    return tt == 1 ? pick(I1(), (f16)0) : tt == 2 ? pick(I2(), (f16)0) : pick(I4(), (f16)0);
  } else if constexpr (MODE == 3) {
    auto pick = [&](auto ttc, auto yt) -> hipError_t {
      constexpr int TT = decltype(ttc)::value;
      using YT = decltype(yt);
      // one tile per workgroup at every N: the persistent loop with the next tile's two
      // matrices in flight measured slower once the tiles outnumber the resident
      // workgroups (MLX K 3072 N 8192 M = 16: 28.0 against 19.5 us)
      return go(k_gemv_xs<P, 3, 8, TT, 1, false, YT>, false);
    };
    if (j.y_f32) return tt == 1 ? pick(I1(), 0.f) : tt == 2 ? pick(I2(), 0.f) : pick(I4(), 0.f);
    return tt == 1 ? pick(I1(), (f16)0) : tt == 2 ? pick(I2(), (f16)0) : pick(I4(), (f16)0);
  } else {
    auto pick = [&](auto ttc) -> hipError_t {
      constexpr int TT = decltype(ttc)::value;
      if constexpr (MODE == 2 && P::WIDE) {
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
