// Device-side building blocks shared by the gfx950 attention kernels.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, the
// v_mfma_f32_16x16x32_{bf16,f16} matrix instructions with fp32 accumulation,
// and LDS tiles padded by 16 bytes per row so that 16-byte fragment reads
// from 16 different rows land in disjoint bank groups.
//
// MFMA fragment convention used by every kernel (16x16x32 shape):
//   lane = lr + 16*lg  (lr = lane & 15, lg = lane >> 4)
//   A operand  (16 rows x 32 k):  lane supplies row lr, k = 8*lg .. 8*lg+7
//   B operand  (32 k x 16 cols):  lane supplies col lr, k = 8*lg .. 8*lg+7
//   C/D (16x16 fp32):             lane holds rows 4*lg .. 4*lg+3 of col lr
// Only the pairing "A register e of lane group lg <-> B register e of lane
// group lg" matters for a contraction, so the kernels are free to permute
// which contraction index sits in which (lg, e) slot as long as both
// operands use the same permutation.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>

namespace farope {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;

// Element-type codes; identical to farope_dtype in include/farope.h.
enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

// ---------------------------------------------------------------------------
// Global-memory I/O of the user tensors (fp32 / fp16 / bf16).
// `vec` is decided on the host: the d-stride is 1 and every base/row offset
// keeps the 16-byte alignment the vector path needs.  Otherwise the generic
// strided path is used (stride 0 is legal, e.g. dO of o.sum()).
// ---------------------------------------------------------------------------
template <typename IO>
__device__ __forceinline__ void load8(const IO* __restrict__ p, int64_t sd, bool vec,
                                      float (&x)[8]) {
  if (vec) {
    if constexpr (sizeof(IO) == 4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(p);
      const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[4 + e] = b[e]; }
    } else {
      typedef IO io8 __attribute__((ext_vector_type(8)));
      const io8 a = *reinterpret_cast<const io8*>(p);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (float)a[e];
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)p[e * sd];
  }
}

// Raw 8-element row segment kept in its I/O type while a load is in flight
// (prefetch registers: 16 bytes for 2-byte types).
template <typename IO> struct Raw8 {
  typedef IO vec __attribute__((ext_vector_type(8)));
  vec v;
};

template <typename IO>
__device__ __forceinline__ Raw8<IO> load_raw8(const IO* __restrict__ p, int64_t sd, bool vec) {
  Raw8<IO> r;
  if (vec) {
    r.v = *reinterpret_cast<const typename Raw8<IO>::vec*>(p);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = p[e * sd];
  }
  return r;
}

template <typename IO>
__device__ __forceinline__ Raw8<IO> zero_raw8() {
  Raw8<IO> r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r.v[e] = (IO)0.f;
  return r;
}

template <typename IO>
__device__ __forceinline__ void unpack8(const Raw8<IO>& r, float (&x)[8]) {
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)r.v[e];
}

template <typename IO>
__device__ __forceinline__ void store4(IO* __restrict__ p, int64_t sd, bool vec,
                                       const float (&x)[4]) {
  if (vec) {
    if constexpr (sizeof(IO) == 4) {
      f32x4 a;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = x[e];
      *reinterpret_cast<f32x4*>(p) = a;
    } else {
      typedef IO io4 __attribute__((ext_vector_type(4)));
      io4 a;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = (IO)x[e];
      *reinterpret_cast<io4*>(p) = a;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e * sd] = (IO)x[e];
  }
}

// ---------------------------------------------------------------------------
// Buffer (descriptor) access for vectorisable tensors: a 128-bit resource in
// SGPRs holds the base address and the byte size of the addressed range; each
// lane supplies a 32-bit byte offset and the wave a uniform one, so no 64-bit
// address arithmetic runs per lane.  Loads past the range return 0 and stores
// past it are dropped.
// ---------------------------------------------------------------------------
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
constexpr int kBufWord3 = 0x00020000;   // raw buffer, 32-bit data format (gfx9 family)

// The base and size must be wave-uniform.  The size passes through
// readfirstlane so that the descriptor is built in SGPRs even where the
// compiler holds the uniform value in VGPRs; a descriptor in VGPRs turns every
// access through it into a loop over the distinct lane values.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           __builtin_amdgcn_readfirstlane((int)bytes), kBufWord3);
}

// 8 elements at byte offset voff + soff
template <typename IO>
__device__ __forceinline__ Raw8<IO> buf_load8(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
  Raw8<IO> x;
  if constexpr (sizeof(IO) == 2) {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    __builtin_memcpy(&x, &a, 16);
  } else {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(r, voff + 16, soff, 0);
    __builtin_memcpy(&x, &a, 16);
    __builtin_memcpy(reinterpret_cast<char*>(&x) + 16, &b, 16);
  }
  return x;
}

// 16-byte buffer store.  A buffer store reads its data VGPRs after it
// issues, so a VALU write to them needs a wait state in between; the
// compiler inserts it only when the store's soffset is an inline constant,
// and with an SGPR soffset it can place the write directly behind the store,
// which then stores the new value (measured on gfx950: dK rows of the
// one-pass backward with fp32 I/O changed from run to run).  The s_nop takes
// the data as an operand: as a side-effecting statement it stays behind the
// store, and the registers cannot be rewritten before it.
__device__ __forceinline__ void buf_store16(u32x4 w, __amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_buffer_store_b128(w, r, voff, soff, 0);
  asm volatile("s_nop 0" : : "v"(w));
}

// 4 elements (converted to IO) at byte offset voff + soff
template <typename IO>
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff,
                                           const float (&x)[4]) {
  if constexpr (sizeof(IO) == 2) {
    typedef IO io4 __attribute__((ext_vector_type(4)));
    io4 a;
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = (IO)x[e];
    u32x2 w;
    __builtin_memcpy(&w, &a, 8);
    __builtin_amdgcn_raw_buffer_store_b64(w, r, voff, soff, 0);
  } else {
    u32x4 w;
    __builtin_memcpy(&w, x, 16);
    buf_store16(w, r, voff, soff);
  }
}

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ...
// lds): the wave's 64 x 16 bytes land at lds + 16 * lane.  The LDS address
// (M0) must be wave-uniform.  Like any buffer load, lanes outside the range
// read zeros.  (A plain function: referenced from a kernel template, the
// builtin would keep the host pass from emitting that kernel's launch stub.)
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* lds, unsigned voff, unsigned soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

// ---------------------------------------------------------------------------
// RoPE.  The packed table is fp32 [(n_pos + 1)][D/2][2] = (cos, sin) per pair;
// row 0 is the identity (cos 1, sin 0) and serves the CLS token, so token s
// uses row s + (1 - has_cls) with no branch.
// ---------------------------------------------------------------------------
// Load (cos, sin) of pairs p0 .. p0+3 of one table row: cs = c0 s0 c1 s1 ...
__device__ __forceinline__ void rope_load4(const float* __restrict__ tab, int row, int d2,
                                           int p0, float (&cs)[8]) {
  const f32x4* t = reinterpret_cast<const f32x4*>(tab + ((int64_t)row * d2 + p0) * 2);
  const f32x4 a = t[0], b = t[1];
#pragma unroll
  for (int e = 0; e < 4; ++e) { cs[e] = a[e]; cs[4 + e] = b[e]; }
}

// x-hat = R x for 4 adjacent pairs (2p, 2p+1):
//   e' = e*c - o*s,  o' = o*c + e*s
__device__ __forceinline__ void rope_rotate8(float (&x)[8], const float (&cs)[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float e = x[2 * p], o = x[2 * p + 1], c = cs[2 * p], s = cs[2 * p + 1];
    x[2 * p] = e * c - o * s;
    x[2 * p + 1] = o * c + e * s;
  }
}

// Gradient through the rotation: g = R^T g-hat for 2 adjacent pairs.
//   ge = ge'*c + go'*s,  go = -ge'*s + go'*c
__device__ __forceinline__ void rope_unrotate4(float (&g)[4], const float* __restrict__ tab,
                                               int row, int d2, int p0) {
  const f32x4 t = *reinterpret_cast<const f32x4*>(tab + ((int64_t)row * d2 + p0) * 2);
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const float e = g[2 * p], o = g[2 * p + 1], c = t[2 * p], s = t[2 * p + 1];
    g[2 * p] = e * c + o * s;
    g[2 * p + 1] = o * c - e * s;
  }
}

// ---------------------------------------------------------------------------
// Transposed fragment reads from row-major LDS tiles (gfx950
// ds_read_b64_tr_b16).  Within each 16-lane group, result lane i, element e
// is 16-bit element (i % 4) of the 8 bytes addressed by lane 4e + i/4 of the
// same group.  So if lane (lr, lg) addresses row R(lg) + lr/4, column
// c0 + 4*(lr % 4) of a row-major tile M, it receives M[R(lg) + e][c0 + lr]
// for e = 0..3: four consecutive rows of one column.  Two such reads (rows
// R and R') give the 8 k-slots of an MFMA operand whose k index runs down
// the columns of M, i.e. a fragment of M^T, without a transposed copy.
// ---------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ s16x4 lds_tr4(const void* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
}

// Physical LDS row of row r of the forward's V tile and of the dK/dV kernel's
// staged Q-hat / dO tiles (16-bit, pitch D + 8 elements): within each 16-row
// half c of a 32-row block, r = 16c + 8a + 4h + i is stored at
// 16c + 2 (i%2 + 2a + 4 (i/2)) + h.  Timed on gfx950, this runs the 16-byte
// operand-row reads of the dK/dV kernel (rows 8 (l/4) + 4h + l%4 of 16
// lanes) at the conflict-free rate instead of 1.45x, and its transposed reads
// at 1.35x instead of 1.0x; in that kernel the trade measured -3.3% of the
// backward.  (For the forward's V, which has only the transposed reads, it
// measured neutral.)
__device__ __forceinline__ int vperm(int r) {
  const int i = r & 3, h = (r >> 2) & 1, a = (r >> 3) & 1;
  return (r & ~15) | (2 * ((i & 1) + 2 * a + 4 * (i >> 1)) + h);
}

// Element offset, inside a row-major tile of pitch `ld`, that lane (lr, lg)
// addresses so that the read yields rows r0 + e (e = 0..3) of column c0 + lr.
__device__ __forceinline__ int tr_offset(int r0, int c0, int ld, int lr) {
  return (r0 + (lr >> 2)) * ld + c0 + 4 * (lr & 3);
}

// ---------------------------------------------------------------------------
// Compute-type traits: how values are kept in LDS and fed to the MFMA unit.
//   DT_BF16: bf16 storage, one v_mfma_f32_16x16x32_bf16 per product.
//   DT_F16 : fp16 storage, one v_mfma_f32_16x16x32_f16 per product.
//   DT_F32 : fp32 storage; each operand is split x = hi + lo (both bf16) and a
//            product is hi*hi + hi*lo + lo*hi (three bf16 MFMAs), about 16
//            mantissa bits, i.e. more than TF32.
// ---------------------------------------------------------------------------
template <int CT> struct Comp;

template <> struct Comp<DT_BF16> {
  typedef bf16 S;
  struct Frag { bf16x8 v; };
  static __device__ __forceinline__ Frag make(const float (&x)[8]) {
    Frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f.v[e] = (bf16)x[e];
    return f;
  }
  static __device__ __forceinline__ Frag zero() { Frag f; f.v = bf16x8{}; return f; }
  static __device__ __forceinline__ void set(Frag& f, int e, float x) { f.v[e] = (bf16)x; }
  // elements 2w, 2w+1 from two floats (one packed conversion)
  static __device__ __forceinline__ void set2(Frag& f, int w, float a, float b) {
    typedef bf16 v2 __attribute__((ext_vector_type(2)));
    v2 t;
    t[0] = (bf16)a;
    t[1] = (bf16)b;
    f.v[2 * w] = t[0];
    f.v[2 * w + 1] = t[1];
  }
  static __device__ __forceinline__ void put_elem(S* p, const Frag& f, int e) { *p = f.v[e]; }
  static __device__ __forceinline__ Frag lds(const S* p) {
    Frag f; f.v = *reinterpret_cast<const bf16x8*>(p); return f;
  }
  // k-slots 0..3 from the transposed read at p0, 4..7 from the one at p1
  static __device__ __forceinline__ Frag tr(const S* p0, const S* p1) {
    const s16x4 a = lds_tr4(p0), b = lds_tr4(p1);
    const s16x8 c = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    Frag f; f.v = __builtin_bit_cast(bf16x8, c); return f;
  }
  // store k-slots 4h..4h+3 (8 bytes)
  static __device__ __forceinline__ void put4(S* p, const Frag& f, int h) {
    typedef S v4 __attribute__((ext_vector_type(4)));
    v4 t;
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = f.v[4 * h + e];
    *reinterpret_cast<v4*>(p) = t;
  }
  static __device__ __forceinline__ void put8(S* p, const float (&x)[8]) {
    *reinterpret_cast<bf16x8*>(p) = make(x).v;
  }
  static __device__ __forceinline__ void put1(S* p, float x) { *p = (bf16)x; }
  static __device__ __forceinline__ f32x4 mma(const Frag& a, const Frag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
  }
};

template <> struct Comp<DT_F16> {
  typedef f16 S;
  struct Frag { f16x8 v; };
  static __device__ __forceinline__ Frag make(const float (&x)[8]) {
    Frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f.v[e] = (f16)x[e];
    return f;
  }
  static __device__ __forceinline__ Frag zero() { Frag f; f.v = f16x8{}; return f; }
  static __device__ __forceinline__ void set(Frag& f, int e, float x) { f.v[e] = (f16)x; }
  static __device__ __forceinline__ void set2(Frag& f, int w, float a, float b) {
    typedef f16 v2 __attribute__((ext_vector_type(2)));
    v2 t;
    t[0] = (f16)a;
    t[1] = (f16)b;
    f.v[2 * w] = t[0];
    f.v[2 * w + 1] = t[1];
  }
  static __device__ __forceinline__ void put_elem(S* p, const Frag& f, int e) { *p = f.v[e]; }
  static __device__ __forceinline__ Frag lds(const S* p) {
    Frag f; f.v = *reinterpret_cast<const f16x8*>(p); return f;
  }
  // k-slots 0..3 from the transposed read at p0, 4..7 from the one at p1
  static __device__ __forceinline__ Frag tr(const S* p0, const S* p1) {
    const s16x4 a = lds_tr4(p0), b = lds_tr4(p1);
    const s16x8 c = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    Frag f; f.v = __builtin_bit_cast(f16x8, c); return f;
  }
  // store k-slots 4h..4h+3 (8 bytes)
  static __device__ __forceinline__ void put4(S* p, const Frag& f, int h) {
    typedef S v4 __attribute__((ext_vector_type(4)));
    v4 t;
#pragma unroll
    for (int e = 0; e < 4; ++e) t[e] = f.v[4 * h + e];
    *reinterpret_cast<v4*>(p) = t;
  }
  static __device__ __forceinline__ void put8(S* p, const float (&x)[8]) {
    *reinterpret_cast<f16x8*>(p) = make(x).v;
  }
  static __device__ __forceinline__ void put1(S* p, float x) { *p = (f16)x; }
  static __device__ __forceinline__ f32x4 mma(const Frag& a, const Frag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, b.v, c, 0, 0, 0);
  }
};

template <> struct Comp<DT_F32> {
  typedef float S;
  struct Frag { bf16x8 h, l; };
  static __device__ __forceinline__ Frag make(const float (&x)[8]) {
    Frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bf16 h = (bf16)x[e];
      f.h[e] = h;
      f.l[e] = (bf16)(x[e] - (float)h);
    }
    return f;
  }
  static __device__ __forceinline__ Frag zero() { Frag f; f.h = bf16x8{}; f.l = bf16x8{}; return f; }
  static __device__ __forceinline__ void set(Frag& f, int e, float x) {
    const bf16 h = (bf16)x;
    f.h[e] = h;
    f.l[e] = (bf16)(x - (float)h);
  }
  static __device__ __forceinline__ void set2(Frag& f, int w, float a, float b) {
    set(f, 2 * w, a);
    set(f, 2 * w + 1, b);
  }
  static __device__ __forceinline__ void put_elem(S* p, const Frag& f, int e) {
    *p = (float)f.h[e] + (float)f.l[e];
  }
  static __device__ __forceinline__ Frag lds(const S* p) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
    float x[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) { x[e] = a[e]; x[4 + e] = b[e]; }
    return make(x);
  }
  static __device__ __forceinline__ void put8(S* p, const float (&x)[8]) {
    f32x4 a, b;
#pragma unroll
    for (int e = 0; e < 4; ++e) { a[e] = x[e]; b[e] = x[4 + e]; }
    *reinterpret_cast<f32x4*>(p) = a;
    *reinterpret_cast<f32x4*>(p + 4) = b;
  }
  static __device__ __forceinline__ void put1(S* p, float x) { *p = x; }
  static __device__ __forceinline__ f32x4 mma(const Frag& a, const Frag& b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.l, b.h, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.l, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.h, b.h, c, 0, 0, 0);
  }
};

// ---------------------------------------------------------------------------
// Split bf16 operands (dS at bf16 compute, head_dim >= 128): x = hi + lo with
// hi = bf16(x) and lo = bf16(x - hi), about 16 significant bits between them.
// A product a.b is then taken as a_hi.b_hi + a_lo.b_hi + a_hi.b_lo (the
// dropped a_lo.b_lo is below the fp32 accumulation error); with one operand
// split only, as a_hi.b_hi + a_hi.b_lo.
// ---------------------------------------------------------------------------
// Pairs: one packed conversion rounds both values; their fp32 images are the
// packed word's low half shifted up and its high half masked (bf16 is the top
// half of an fp32), so hi, lo of two values cost 6 VALU instructions.
__device__ __forceinline__ void split_bf16x8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef bf16 b2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const b2 h = __builtin_convertvector(f2{x[2 * p], x[2 * p + 1]}, b2);
    const unsigned u = __builtin_bit_cast(unsigned, h);
    const float h0 = __uint_as_float(u << 16), h1 = __uint_as_float(u & 0xffff0000u);
    const b2 l = __builtin_convertvector(f2{x[2 * p] - h0, x[2 * p + 1] - h1}, b2);
    hi[2 * p] = h[0];
    hi[2 * p + 1] = h[1];
    lo[2 * p] = l[0];
    lo[2 * p + 1] = l[1];
  }
}

// ---------------------------------------------------------------------------
// fp16 logit operands (bf16 compute at head_dim >= 128): the rotated Q / K
// rows enter the logits product rounded to fp16 (11 significant bits against
// bf16's 8), one MFMA per product.  fp16 ends at 65504 and has normal values
// down to 2^-14 only, so each kernel keeps the largest |x| it converts.  When
// a tile's Q-hat or K-hat reaches 2^12 -- past that fp16 could overflow, or
// the other operand's values in fp16's subnormal range could shift a logit by
// more than 128 * 2^-25 * 2^12 = 2^-6 -- the tile is computed once more with
// both operands scaled by f16_fit (powers of two that put each maximum in
// [2^14, 2^15)) and the logits multiplied by the inverse scales in fp32.
// Otherwise the scales are 1 and the factor is exact.
// ---------------------------------------------------------------------------
constexpr unsigned kF16ExpLimit = 139;   // biased fp32 exponent of 2^12
constexpr unsigned kF16ExpLow = 117;     // biased fp32 exponent of 2^-10

// running max of |x| over 8 values (NaN is ignored)
__device__ __forceinline__ float amax8(float a, const float (&x)[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) a = fmaxf(a, fmaxf(fabsf(x[2 * p]), fabsf(x[2 * p + 1])));
  return a;
}
// fp16 images of 8 values, two per packed conversion (round to nearest even)
__device__ __forceinline__ f16x8 to_f16x8(const float (&x)[8]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef f16 h2 __attribute__((ext_vector_type(2)));
  f16x8 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const h2 h = __builtin_convertvector(f2{x[2 * p], x[2 * p + 1]}, h2);
    r[2 * p] = h[0];
    r[2 * p + 1] = h[1];
  }
  return r;
}
// Operand scale of a rescaled pass for a maximum |x| with biased exponent e:
// 2^(141 - e), which puts the scaled maximum in [2^14, 2^15), at most 2^64
// (an operand that small contributes nothing a logit could resolve).
// e = 255 (inf) gives 2^-114, which leaves inf as inf: such inputs end as
// inf / NaN, as they do in fp32 arithmetic.
__device__ __forceinline__ float f16_fit(unsigned e) {
  return __uint_as_float((e >= 77u ? 268u - e : 191u) << 23);
}

// ---------------------------------------------------------------------------
// Misc.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Sum / max over the 4 lane groups that share one MFMA column (lanes
// lr, lr+16, lr+32, lr+48), with the gfx950 row-swap instructions (VALU, no
// LDS round trip).  v_permlane16_swap(x, x) returns {x', x''} where, for
// every lane, one of the two is the lane's own x and the other the x of
// lane ^ 16; v_permlane32_swap does the same for lane ^ 32.  A commutative
// op over the pair therefore combines each lane with its partner.
__device__ __forceinline__ float xor16_pair_op_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_pair_op_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_pair_op_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_pair_op_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float group4_sum(float v) { return xor32_pair_op_sum(xor16_pair_op_sum(v)); }
__device__ __forceinline__ float group4_max(float v) { return xor32_pair_op_max(xor16_pair_op_max(v)); }

// Largest of a non-negative float over the wave, as its fp32 bit pattern
// (those order like the values), in every lane: DPP within each 16-lane row
// (both quad permutations, then the mirror images within the half row and
// the row), then the two row swaps -- VALU only, no LDS round trip.
__device__ __forceinline__ unsigned wave_max_bits(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false)));
  return __float_as_uint(group4_max(x));
}

// Work-item / workgroup ids straight from the hardware registers.  (The
// threadIdx / blockIdx / gridDim accessors are device-library calls, and the
// kernels here are built with IEEE mode off, which that library is not, so
// they would not be inlined: every use would become a real call with a stack
// frame.  The launch grid size is passed in the kernel arguments instead.)
__device__ __forceinline__ int thread_id() { return __builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int block_id() { return __builtin_amdgcn_workgroup_id_x(); }

// Workgroups are dispatched round-robin over MI355X's 8 XCDs (each with its
// own L2).  Remap the linear workgroup id so that XCD x processes one
// contiguous range of tiles; consecutive tiles (the q/kv blocks of one
// (b, h) plane) then share that XCD's L2.  Bijective for any total T.
__device__ __forceinline__ int xcd_remap(int L, int T) {
  constexpr int X = 8;
  const int per = T / X, rem = T % X;
  const int x = L % X, i = L / X;
  return x * per + (x < rem ? x : rem) + i;
}

__device__ __forceinline__ int round_up32(int x) { return (x + 31) & ~31; }

// sum_e a[e] * b[e] over an 8-element row segment, plus c, in fp32.  16-bit
// types use the packed dot instructions (v_dot2c_f32_{bf16,f16}) on the raw
// registers; the products of 16-bit values are exact in fp32 either way.
template <typename IO>
__device__ __forceinline__ float dot8(const Raw8<IO>& a, const Raw8<IO>& b, float c) {
  if constexpr (sizeof(IO) == 2) {
    typedef IO io2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const io2 x = {a.v[2 * e], a.v[2 * e + 1]}, y = {b.v[2 * e], b.v[2 * e + 1]};
      if constexpr (std::is_same<IO, bf16>::value)
        c = __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
      else
        c = __builtin_amdgcn_fdot2(x, y, c, false);
    }
    return c;
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) c = __builtin_fmaf((float)a.v[e], (float)b.v[e], c);
    return c;
  }
}

// Sum over each aligned group of 8 consecutive lanes, result in every lane of
// the group.  DPP moves inside a row (no LDS traffic): swap neighbours, swap
// pairs (both quad permutations), then add the mirror image within the
// 8-lane half row, which pairs each lane with one of the other quad.
__device__ __forceinline__ float dpp_sum8(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));   // quad_perm 1,0,3,2
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));   // quad_perm 2,3,0,1
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
  return x;
}

// A copy of x the compiler cannot see through.  Index math derived from it is
// recomputed where it is used instead of being hoisted out of the enclosing
// loops, which keeps per-lane addresses of rarely run phases (per-plane
// prologue / epilogue) from occupying registers through the hot loop.
__device__ __forceinline__ int opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}
// The same for a float: pins a value computed early (a running maximum of
// converted operands) where it is computed, instead of letting its inputs
// stay live until the value's only use at the end of a tile.
__device__ __forceinline__ float opaque(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

// The same for a 16-byte register vector (an MFMA operand fragment): values
// computed from it after a loop are formed there, not kept from before it.
template <typename V>
__device__ __forceinline__ V opaque_vec(V x) {
  asm volatile("" : "+v"(x));
  return x;
}

// Workgroup barrier that orders LDS traffic only.  The waves of these kernels
// exchange data through LDS alone, so the barrier waits for outstanding LDS
// operations (lgkmcnt) but not for global loads and stores (vmcnt): prefetches
// of the next tile and stores of finished results stay in flight across it.
// (__syncthreads() would drain every outstanding global access first.)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace farope
