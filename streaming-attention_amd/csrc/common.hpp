// Shared device helpers for the streaming Taylor+coreset attention kernels (gfx950 / CDNA4).
//
// Conventions used by every kernel in this library:
//   * q, k, v are contiguous [BH, N, D] / [BH, N, Dv] tensors in fp32, bf16 or fp16; all arithmetic
//     is fp32 (scores for the block compressor are accumulated in fp64).
//   * Matrix-core work uses v_mfma_f32_16x16x4_f32 (64-wide wavefront).  Operand layouts, for a lane
//     l = 16*g + i (i = l % 16, g = l / 16):
//         A (16x4):  lane holds A[i][g]
//         B (4x16):  lane holds B[g][i]
//         D (16x16): lane holds D[4*g + r][i] in element r of the float4 accumulator.
//     A D-tile produced by one MFMA is re-used as the B operand of the next contraction without any
//     data movement by visiting the contraction index in the order {4*g + s}, s = 0..3: for K-step s
//     the B value lane l needs is exactly element s of its own accumulator.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sta {

typedef float floatx4 __attribute__((ext_vector_type(4)));

enum DType : int { F32 = 0, BF16 = 1, F16 = 2 };

__device__ __forceinline__ float load_elem(const void* base, int64_t idx, int dtype) {
  if (dtype == F32) return static_cast<const float*>(base)[idx];
  if (dtype == BF16) {
    uint32_t bits = static_cast<uint32_t>(static_cast<const uint16_t*>(base)[idx]) << 16;
    return __uint_as_float(bits);
  }
  return static_cast<float>(static_cast<const _Float16*>(base)[idx]);
}

__device__ __forceinline__ void store_elem(void* base, int64_t idx, int dtype, float x) {
  if (dtype == F32) {
    static_cast<float*>(base)[idx] = x;
  } else if (dtype == BF16) {
    // round-to-nearest-even, NaN kept quiet
    uint32_t u = __float_as_uint(x);
    uint16_t h;
    if ((u & 0x7fffffffu) > 0x7f800000u) {
      h = static_cast<uint16_t>((u >> 16) | 0x40u);
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
      h = static_cast<uint16_t>(u >> 16);
    }
    static_cast<uint16_t*>(base)[idx] = h;
  } else {
    static_cast<_Float16*>(base)[idx] = static_cast<_Float16>(x);
  }
}

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Buffer resource of raw memory at p (stride 0, the largest record count, the gfx9 data-format word):
// a buffer access addresses base + a per-lane 32-bit offset + a uniform 32-bit offset, so a loop
// whose per-lane offsets are invariant and whose uniform offset advances needs no per-lane 64-bit
// address arithmetic.  Callers keep every offset sum below 2^32 and inside their own allocation.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, -1, 0x00020000);
}
// the cache-policy operand of a non-temporal buffer store
constexpr int BUF_NT = 2;

// Split-bf16 products (bf16 matrix cores at 16x the fp32 rate).  An fp32 value x is carried as
// hi = bf16(x) and lo = bf16(x - hi), both rounded to nearest even: x - hi is exact in fp32 and
// |x - hi - lo| <= 2^-9 |x - hi| <= 2^-18 |x|.  A product is taken as hi.hi' + hi.lo' + lo.hi' (bf16
// products are exact, sums fp32), which drops lo.lo' (<= 2^-18 |x x'|): about 2^-16 relative error
// per product, against 2^-11 for the tf32 operands of the reference's Triton dots.
// v_mfma_f32_16x16x32_bf16, lane l = 16 g + i:  A[i][8 g + j] = a[j],  B[8 g + j][i] = b[j],
// D[4 g + r][i] = d[r]  (the layout of mfma4 with 8 contraction elements per lane instead of one).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ floatx4 mfma_bf16(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// two floats to packed bf16 (one v_cvt_pk_bf16_f32, round to nearest even)
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){a, b}, bf16x2));
}

// hi and lo of two values as packed bf16 pairs in 4 VALU: packed hi (v_cvt_pk_bf16_f32), x - hi with
// one v_dot2_f32_bf16 per value, packed lo.  The dot product of the packed hi pair with the bf16 pair
// (-1, 0) (or (0, -1)) plus x is x - hi exactly: bf16 products are exact in fp32 and x - hi is
// representable.  The two pairs are held in scalar registers behind an empty asm: the compiler would
// otherwise encode (-1, 0) as the inline constant -1.0, which the hardware reads as the 32-bit float
// (the pair (0, -1)).  The dot stays the compiler's builtin (selected as v_dot2c_f32_bf16, which costs
// a v_mov where x stays live): a VALU instruction written as inline asm is invisible to the compiler's
// MFMA hazard padding, and such a form gave wrong moments next to the matrix-core products.
__device__ __forceinline__ void split_pair(float a, float b, uint32_t& h, uint32_t& l) {
  // a pair the optimiser knows to be zero (the padding half of an odd tile pair) costs nothing
  if (__builtin_constant_p(a) && __builtin_constant_p(b) && a == 0.f && b == 0.f) {
    h = l = 0u;
    return;
  }
  uint32_t c0 = 0x0000BF80u, c1 = 0xBF800000u;
  asm("" : "+s"(c0));
  asm("" : "+s"(c1));
  const bf16x2 hp = __builtin_convertvector((floatx2){a, b}, bf16x2);
  h = __builtin_bit_cast(uint32_t, hp);
  l = pk_bf16(__builtin_amdgcn_fdot2_f32_bf16(hp, __builtin_bit_cast(bf16x2, c0), a, false),
              __builtin_amdgcn_fdot2_f32_bf16(hp, __builtin_bit_cast(bf16x2, c1), b, false));
}

__device__ __forceinline__ void split_bf16(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) split_pair(x[2 * p], x[2 * p + 1], h[p], l[p]);
  hi = __builtin_bit_cast(bf16x8, uint4{h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(bf16x8, uint4{l[0], l[1], l[2], l[3]});
}

// c += a.b for split operands (three bf16 matrix-core products)
__device__ __forceinline__ floatx4 mfma_split(const bf16x8& ah, const bf16x8& al, const bf16x8& bh,
                                              const bf16x8& bl, floatx4 c) {
  c = mfma_bf16(ah, bl, c);
  c = mfma_bf16(al, bh, c);
  return mfma_bf16(ah, bh, c);
}

// Empty register constraint: pins the computation of x at this point of the instruction stream (keeps
// the scheduler from sinking an accumulation chain and holding all of its inputs live).
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

// Taylor truncation sum_{r<=deg} x^r / r!, evaluated term by term (term = term * x / r) so that the
// fp32 rounding sequence is the one of the reference's exp_taylor.
__device__ __forceinline__ float taylor_poly(float x, int deg) {
  float out = 1.0f;
  float term = 1.0f;
  for (int r = 1; r <= deg; ++r) {
    term = __fdiv_rn(__fmul_rn(term, x), static_cast<float>(r));
    out = __fadd_rn(out, term);
  }
  return out;
}

// Elements [off, off+4) of a row as raw bits: 16 bytes (ES = 4) or 8 bytes (ES = 2, in .x/.y).  Rows are
// read in units of 4 elements; the caller guarantees alignment and that the unit lies in the row.
template <int ES>
__device__ __forceinline__ uint4 load_unit(const void* base, int64_t off) {
  if constexpr (ES == 4) {
    return *reinterpret_cast<const uint4*>(static_cast<const float*>(base) + off);
  } else {
    const uint2 r = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(base) + off);
    return uint4{r.x, r.y, 0u, 0u};
  }
}

// A raw unit as 4 floats (fp32 bits when ES = 4, else bf16 / fp16 by dtype), times `scale`.
template <int ES>
__device__ __forceinline__ floatx4 unit_to_f4(const uint4& r, int dtype, float scale) {
  floatx4 f;
  if constexpr (ES == 4) {
    f = floatx4{__uint_as_float(r.x), __uint_as_float(r.y), __uint_as_float(r.z), __uint_as_float(r.w)};
  } else if (dtype == BF16) {
    f = floatx4{__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u), __uint_as_float(r.y << 16),
                __uint_as_float(r.y & 0xffff0000u)};
  } else {
    f = floatx4{static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.x & 0xffffu))),
                static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.x >> 16))),
                static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.y & 0xffffu))),
                static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r.y >> 16)))};
  }
  return f * scale;
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup w runs on XCD w % 8).  This maps
// the hardware workgroup id to a logical id such that consecutive logical ids share an XCD, so the
// workgroups that read the same head's rows share one L2.
__device__ __forceinline__ int xcd_remap(int wg, int total) {
  if ((total & 7) != 0) return wg;
  return (wg & 7) * (total >> 3) + (wg >> 3);
}

}  // namespace sta
