// Shared device helpers for the emx_attn kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emx {

typedef _Float16 h16;
typedef h16 h16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kTwo24 = 16777216.0f;  // codes enter the MFMA as fp16 subnormals n * 2^-24

// One LDS arena that the 4-bit decode and the prefill kernel bodies carve their
// arrays from.  A kernel allocates every __shared__ variable it references, so
// the two bodies of one launch (unified_q4) overlap in it instead of adding up;
// either kernel alone takes the arena's size.
constexpr int kArenaBytes = 62 * 1024;
__shared__ __attribute__((aligned(16))) unsigned char lds_arena[kArenaBytes];

// The object of type T at byte offset off of the arena.
template <class T>
__device__ __forceinline__ T& lds_at(const int off) {
  return *reinterpret_cast<T*>(lds_arena + off);
}
// Offset after an object of `bytes` at `off`, 16-byte aligned.
constexpr int lds_next(const int off, const int bytes) { return (off + bytes + 15) & ~15; }

__device__ __forceinline__ h16x8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  u32x4 v = {a, b, c, d};
  return __builtin_bit_cast(h16x8, v);
}

// One uint32 of eight 4-bit codes -> eight exact fp16 subnormals (code * 2^-24).
// Element order: (n0, n4, n1, n5, n2, n6, n3, n7).
__device__ __forceinline__ h16x8 unpack4(uint32_t w) {
  return as_h8(w & 0x000F000Fu, (w >> 4) & 0x000F000Fu, (w >> 8) & 0x000F000Fu, (w >> 12) & 0x000F000Fu);
}

// Two uint32 of four 8-bit codes each -> eight exact fp16 subnormals, in order.
__device__ __forceinline__ h16x8 unpack8(uint32_t w0, uint32_t w1) {
  return as_h8(__builtin_amdgcn_perm(0u, w0, 0x0C010C00u), __builtin_amdgcn_perm(0u, w0, 0x0C030C02u),
               __builtin_amdgcn_perm(0u, w1, 0x0C010C00u), __builtin_amdgcn_perm(0u, w1, 0x0C030C02u));
}

// Position (0..7 within the 8 codes of one MFMA k-slice) of MFMA element i.
template <int BITS>
__device__ __forceinline__ constexpr int slot_perm(int i) {
  return BITS == 4 ? ((i >> 1) + ((i & 1) << 2)) : i;
}

__device__ __forceinline__ f32x4 mfma16x16x32(h16x8 a, h16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float(((uint32_t)v) << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);  // quiet NaN
  uint32_t r = x + 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(r >> 16);
}

// Element type tags for the dense (unquantized) cache path.
struct F16 { typedef h16 T; };
struct BF16 { typedef uint16_t T; };
struct F32 { typedef float T; };

__device__ __forceinline__ float to_f32(h16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(uint16_t v) { return bf16_to_f32(v); }
__device__ __forceinline__ void from_f32(float f, h16* p) { *p = (h16)f; }
__device__ __forceinline__ void from_f32(float f, float* p) { *p = f; }
__device__ __forceinline__ void from_f32(float f, uint16_t* p) { *p = f32_to_bf16(f); }

// Bit offset of token k inside its value word.  4-bit value words interleave
// their eight tokens, token k at nibble (k >> 1) | ((k & 1) << 2), so that
// masking a word with 0x000F000F / 0x00F000F0 (and the same after >> 8) yields
// the token pairs (0,1), (2,3), (4,5), (6,7) as fp16 subnormals (the second
// and fourth pair scaled by 16).  8-bit value words hold tokens in byte order.
template <int BITS>
__host__ __device__ __forceinline__ constexpr int v_shift(int k) {
  return BITS == 4 ? 4 * (((k & 7) >> 1) | ((k & 1) << 2)) : 8 * (k & 3);
}

// Value pages are stored in tiles of T = min(page_size, 256/BITS) tokens; inside a
// tile they are dim-major with T*BITS/32 words per dim (32 bytes when the page
// holds a whole tile), so one decode iteration's value codes are one contiguous
// 4 KiB block.  Word index of (page-head ph, token off, dim d):
template <int BITS>
__host__ __device__ __forceinline__ size_t v_word_index(size_t ph, int off, int d, int D, int bs) {
  constexpr int TMAX = 256 / BITS;
  const int T = bs < TMAX ? bs : TMAX;
  return ((ph * (size_t)(bs / T) + (size_t)(off / T)) * D + d) * (size_t)(T * BITS / 32) + (off % T) / (32 / BITS);
}

// FP8 E4M3 code -> float, as the reference's kernels decode it
// (lib/python/easymlx/operations/kernels/unified_attention.py:1275-1285): no NaN
// code, exponent 15 with mantissa 7 is (1 + 7/8) * 2^8.
__device__ __forceinline__ float e4m3_to_f32(uint32_t c) {
  const uint32_t e = (c >> 3) & 0xFu, m = c & 0x7u;
  const float v = e == 0 ? (float)m * 0.001953125f : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (c & 0x80u) ? -v : v;
}

// Two E4M3 bytes at bits 0-7 and 16-23 of y (zeros elsewhere) -> two fp16 equal
// to dec(byte) * 2^-8 exactly: the 16-bit value (b + (b & 0x80)) << 7 keeps the
// sign and shifts exponent and mantissa up by seven bits (normals: exponent bias
// 15 against 7; sub-normals: m * 2^-17 = m * 2^-9 * 2^-8; 0x7F gives 1.875 =
// 480 * 2^-8, the reference decoder's value for that code).
__device__ __forceinline__ uint32_t e4m3x2_to_h16x2(const uint32_t y) { return (y + (y & 0x00800080u)) << 7; }

// float -> FP8 E4M3 code with the reference's encoder
// (lib/python/easymlx/operations/kernels/_metal_header.py:339-419): round to
// nearest even for exponents 1..14, round half up through its sub-normal
// branch otherwise (which also takes 240 < |x| <= 448 and keeps only the low
// mantissa bits there), |x| > 448 and infinities to 448, NaN to 0x7F.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  const uint32_t bits = __float_as_uint(f), s = bits >> 31, ab = bits & 0x7FFFFFFFu;
  if (ab > 0x7F800000u) return 0x7Fu;
  if (ab == 0x7F800000u || ab > 0x43E00000u) return (s << 7) | 0x7Eu;  // 0x43E00000 = 448.0f
  const int e8 = (int)((ab >> 23) & 0xFFu) - 120;
  const uint32_t m = ab & 0x7FFFFFu;
  uint32_t r;
  if (e8 >= 1 && e8 <= 14) {
    uint32_t mant = m >> 20;
    const uint32_t lsb = mant & 1u, rnd = (m >> 19) & 1u, sticky = (m & 0x7FFFFu) != 0u;
    mant += rnd & (sticky | lsb);
    int ee = e8;
    if (mant >> 3) {
      mant = 0;
      if (++ee > 14) return (s << 7) | (0xFu << 3);
    }
    r = (s << 7) | ((uint32_t)ee << 3) | (mant & 0x7u);
  } else {
    if (e8 < -2) return s << 7;
    const int rshift = (1 - e8) + 20;
    const uint32_t rounded = ((0x800000u | m) + (1u << (rshift - 1))) >> rshift;
    if (rounded == 0) return s << 7;
    r = (s << 7) | (rounded & 0x7u);
  }
  if (((r >> 3) & 0xFu) == 0xFu && (r & 0x7u) == 0x7u) r = (s << 7) | 0x7Eu;
  return r;
}

// Rotary position embedding as mlx.core.fast.rope rotates for the reference's
// RoPE modules (nn.RoPE; Llama3RoPE / SuScaledRoPE / YarnRoPE pass their own
// frequencies, lib/python/easymlx/layers/rotary/_rotary.py:134-221): pair i of
// the first `rot` dims -- (i, i + rot/2), or (2i, 2i+1) when traditional --
// turns by theta = position * inv_freq[i]; other dims pass through.
struct RopeArgs {
  const float* inv_freq;       // [rot / 2], null: no rotation
  const int32_t* positions;    // [T] position of each token
  int rot;                     // rotated dims (even, <= D)
  int traditional;
};

// sin and cos of a RoPE angle: the rotations below and the (token, pair) tables
// that the fused writes build all take them from here.
__device__ __forceinline__ void rope_sincos(const float theta, float* sn, float* cs) { sincosf(theta, sn, cs); }

// (x0, x1) turned by the angle whose sine and cosine are given: fp32 products
// and sums rounded one by one, so every kernel that rotates gets the same bits.
// (HIP's __fmul_rn and __fadd_rn are plain operators compiled under the
// header's -ffp-contract=fast, which fused a product into the following sum at
// some call sites and not at others; the operators are written here with
// contraction off.)
__device__ __forceinline__ void rope_rotate_sc(const float x0, const float x1, const float2 sc, float& y0, float& y1) {
#pragma clang fp contract(off)
  y0 = x0 * sc.y - x1 * sc.x;
  y1 = x0 * sc.x + x1 * sc.y;
}

// (y0, y1) = (x0, x1) turned by theta (rope_rotate_sc on rope_sincos(theta)).
__device__ __forceinline__ void rope_rotate(const float x0, const float x1, const float theta, float& y0, float& y1) {
  float sn, cs;
  rope_sincos(theta, &sn, &cs);
  rope_rotate_sc(x0, x1, float2{sn, cs}, y0, y1);
}

// Max / sum over the lanes i, i^16, i^32, i^48 (one column of the four 16-lane
// rows, the MFMA output rows of a 16-wide tile) with gfx950's row swaps:
// v_permlane16_swap pairs rows (0,1) and (2,3), v_permlane32_swap the halves.
// Plain VALU, no LDS round trip (a __shfl_xor is a ds_bpermute); every lane of
// a column gets the same bits.
__device__ __forceinline__ float rows4_max(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows4_sum(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

constexpr int kRsrcFlags = 0x00020000;  // raw 32-bit buffer, gfx9 family
constexpr int kLoadAux = 0;             // default cache policy

// Raw buffer descriptor of `bytes` bytes at p, built from wave-uniform values
// moved to SGPRs (a descriptor the compiler keeps in VGPRs makes it wrap every
// load through it in a per-lane loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* p, const int bytes) {
  const uint64_t x = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)x);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(x >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0,
                                           __builtin_amdgcn_readfirstlane(bytes), kRsrcFlags);
}

}  // namespace emx
