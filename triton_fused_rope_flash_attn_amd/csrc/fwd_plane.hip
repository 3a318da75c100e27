// Forward kernel for ViT-sized planes: one wave per (b, h) plane.
//
// Reference behaviour followed: _attn_fwd in "fa_rope_full .py" (FA:91-315):
// Q/K pair rotation with the CLS row bypassing RoPE (FA:176-202, FA:248-272),
// scaled logits with padded key columns masked out (FA:275-277), softmax
// (FA:280-305) and the per-row log-sum-exp stored for the backward pass
// (FA:308-309).
//
// Planes of 193 .. 208 tokens at head_dim 64 with 16-bit tensors (ViT-S/B/L
// at 224 px: 14 x 14 patches + CLS = 197 tokens).  The persistent kernel runs
// one wave per SIMD (4-wave workgroups, up to 512 registers per wave) and each
// wave computes whole planes on its own:
//  * The plane's rotated K-hat (13 tiles of 16 keys x 64 channels) and V^T
//    (4 channel tiles x 7 steps of 32 keys) are loaded once into registers as
//    MFMA A-operands (the compiler keeps them in AGPRs) and serve all 13
//    query subtiles: no LDS traffic, no barrier and no cross-wave dependency
//    in the hot loop.  A plane's 13 subtiles run on one SIMD, so there is no
//    16-row padding subtile per SIMD either.
//  * Logits are computed transposed, S^T = K-hat Q-hat^T, 16 keys x 16
//    queries per MFMA tile: lane (lr, lg) holds keys 16u + 4lg + i of query
//    lr, which is the B-operand layout of O^T += V^T P^T, so P never leaves
//    registers.  All 208 logits of a query row are in registers at once:
//    softmax is single-pass (exact row max, no running rescale).
//  * S of subtile t + 1 is issued before the softmax of subtile t, so the
//    MFMA pipe works while the VALU computes probabilities.
//  * V reaches LDS by direct-to-LDS buffer loads (one wave-private 26 KB
//    buffer) one plane ahead; the transposed fragment reads
//    (ds_read_b64_tr_b16) run once per plane.  The RoPE table is copied to
//    LDS once per workgroup.
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

namespace {
constexpr int kFpW = 4;                      // waves per workgroup (one per SIMD)
constexpr int kFpD = 64;                     // head_dim
constexpr int kFpKT = 13;                    // 16-key tiles: planes of 193 .. 208 tokens
constexpr int kFpRows = 16 * kFpKT;          // padded keys / queries per plane
constexpr int kFpKS = (kFpRows + 31) / 32;   // 32-key steps of O^T = V^T P^T
}  // namespace

// The plane's K-hat / V^T fragments are MFMA A-operands only: an empty asm
// with an AGPR output tied to the value makes the register allocator keep them
// in AGPRs (MFMA reads its A operand from there directly), which leaves the
// VGPRs to the logits, probabilities and accumulators.
template <typename V>
__device__ __forceinline__ V in_agpr(V x) {
  V y;
  asm("" : "=a"(y) : "0"(x));
  return y;
}

bool fwd_plane_ok(int io, int ct, int D, int N, int has_cls, bool vec) {
  // (the LDS table holds kFpRows + 1 rows: every position of such a plane)
  (void)has_cls;
  return vec && D == kFpD && io != DT_F32 && ct == io && N > kFpRows - 16 && N <= kFpRows;
}
int fwd_plane_rows() { return kFpRows; }
int fwd_plane_threads() { return kFpW * 64; }

template <typename IO>
__global__ void __launch_bounds__(kFpW * 64) fwd_plane_kernel(const FwdParams p) {
  constexpr int CT = std::is_same<IO, f16>::value ? DT_F16 : DT_BF16;
  using C = Comp<CT>;
  using Frag = typename C::Frag;
  constexpr int D = kFpD, KT = kFpKT, KS = kFpKS;
  constexpr unsigned ES = sizeof(IO);
  static_assert(ES == 2, "16-bit tensors only");
  // V rows of each wave's plane (row-major, 128-byte rows) and the packed
  // RoPE table (16-byte chunk c of row r at chunk c ^ (r & 15)); table rows
  // past the plane's positions are zero, so the padded rows of the last tile
  // (zero Q / K rows) read finite values without a clamp.
  constexpr int TROWS = kFpRows + 1;
  __shared__ __attribute__((aligned(16))) IO sV[kFpW][kFpRows * D];
  __shared__ __attribute__((aligned(16))) float sTab[TROWS * D];

  const int tid = thread_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int N = p.N, shift = 1 - p.has_cls;
  const float c2 = p.scale_log2;
  const int planes = p.B * p.H;
  IO* const myV = sV[wave];

  {
    const int nrows = N + shift;
    for (int u = tid; u < TROWS * 16; u += kFpW * 64) {
      const int r = u >> 4, c = u & 15;
      f32x4 x = {0.f, 0.f, 0.f, 0.f};
      if (r < nrows) x = *reinterpret_cast<const f32x4*>(p.rope + (int64_t)r * D + 4 * c);
      *reinterpret_cast<f32x4*>(&sTab[(r * 16 + (c ^ (r & 15))) * 4]) = x;
    }
    // V rows N .. kFpRows - 1 of every buffer are never loaded: zero them
    // (their probabilities are 0, and 0 * garbage could be NaN)
    const int zr = kFpRows - N;
    for (int u = tid; u < kFpW * zr * 8; u += kFpW * 64) {
      const int w = u / (zr * 8), x = u - w * (zr * 8);
      *reinterpret_cast<u32x4*>(&sV[w][(N + (x >> 3)) * D + 8 * (x & 7)]) = u32x4{0, 0, 0, 0};
    }
  }
  __syncthreads();

  auto plane_ptr = [&](const void* base, const int64_t* st, int plane) __attribute__((always_inline)) {
    const int bb = plane / p.H, hh = plane - bb * p.H;
    return static_cast<const IO*>(base) + bb * st[0] + hh * st[1];
  };
  auto rsrc = [&](const void* b, const int64_t* st, int plane) __attribute__((always_inline)) {
    return make_rsrc(plane_ptr(b, st, plane), (unsigned)(((int64_t)(N - 1) * st[2] + D) * ES));
  };
  // cos/sin of the lane's 8 channels 32s + 8lg .. +7 (pairs 16s + 4lg ..
  // +3) for row 16t + lr of the plane: table row 16t + lr + shift, whose low
  // four bits (the chunk swizzle) do not depend on t.  The per-lane part of
  // the address is formed once (opaque: not hoisted as 13 separate
  // addresses); t enters as an immediate offset.
  const int trow = lr + shift, tsw = trow & 15;
  const float* tab_lane[2][2];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      tab_lane[s][h] = &sTab[opaque((trow * 16 + ((8 * s + 2 * lg + h) ^ tsw)) * 4)];
  auto tab8 = [&](int t, int s, float (&cs)[8]) __attribute__((always_inline)) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(tab_lane[s][0] + t * 16 * D);
    const f32x4 b = *reinterpret_cast<const f32x4*>(tab_lane[s][1] + t * 16 * D);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      cs[e] = a[e];
      cs[4 + e] = b[e];
    }
  };
  // V rows 0 .. kFpRows-1 of `plane` -> this wave's LDS buffer: each 16-byte
  // direct load of a lane lands at buffer + 16 * lane, i.e. 8 rows per
  // instruction; rows >= N are outside the descriptor's range (not loaded).
  auto dma_row8 = [&](const __amdgpu_buffer_rsrc_t& rV, int i) __attribute__((always_inline)) {
    const unsigned vo = (unsigned)(((lane >> 3) * (int)p.sv[2] + 8 * (lane & 7)) * (int)ES);
    // rows 8i .. 8i + 7; those of the last key tile may be >= N (lane offset)
    const unsigned rows = (unsigned)(8 * i * (int)p.sv[2] * (int)ES);
    const bool last = 8 * i >= 16 * (KT - 1);
    lds_dma16(rV, myV + i * 8 * D, last ? vo + rows : vo, last ? 0u : rows);
  };
  auto dma_v = [&](int plane) __attribute__((always_inline)) {
    const auto rV = rsrc(p.v, p.sv, plane);
#pragma unroll
    for (int i = 0; i < kFpRows / 8; ++i) dma_row8(rV, i);
  };
  // 16-byte row segments (rows 16t + lr, channels 32s + 8lg ..): a per-lane
  // byte offset, plus the tile's first row as a scalar offset.  Only the last
  // tile holds rows >= N; its row offset goes into the lane offset instead, so
  // that those rows fall outside the descriptor's range (the range check
  // covers the lane and instruction offsets).
  const unsigned qoff = (unsigned)opaque((lr * (int)p.sq[2] + 8 * lg) * (int)ES);
  const unsigned koff = (unsigned)opaque((lr * (int)p.sk[2] + 8 * lg) * (int)ES);
  auto tile_off = [&](unsigned voff, int t, int64_t st, unsigned& v, unsigned& so) __attribute__((always_inline)) {
    const unsigned rows = (unsigned)(16 * t * (int)st * (int)ES);
    if (t == KT - 1) {
      v = voff + rows;
      so = 0u;
    } else {
      v = voff;
      so = rows;
    }
  };
  auto load_q = [&](const __amdgpu_buffer_rsrc_t& rQ, int t, Raw8<IO> (&q)[2]) __attribute__((always_inline)) {
    unsigned v, so;
    tile_off(qoff, t, p.sq[2], v, so);
#pragma unroll
    for (int s = 0; s < 2; ++s) q[s] = buf_load8<IO>(rQ, v + 64 * s, so);
  };
  auto rot_q = [&](const Raw8<IO> (&q)[2], int t, Frag (&f)[2]) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float x[8], cs[8];
      unpack8(q[s], x);
      tab8(t, s, cs);
      rope_rotate8(x, cs);
      f[s] = C::make(x);
    }
  };

  // O: lane groups lg, lg ^ 1 trade halves so that each lane stores 8
  // channels 16 (d0 + (lg & 1)) + 4 (lg & 2) .. +7 of row 16t + lr (16 bytes)
  const unsigned ooff = (unsigned)opaque((lr * (int)p.so[2] + 16 * (lg & 1) + 4 * (lg & 2)) * (int)ES);
  const unsigned loff = (unsigned)opaque(lg == 0 ? 4 * lr : 4 * N + 64 * KT);
  // the last key tile's keys >= N are masked (-inf logits)
  const int klim = N - 16 * (KT - 1) - 4 * lg;

  // V^T fragments of the plane in this wave's LDS buffer: k-slot e of lane
  // group lg is key 32j + 4lg + e (e < 4) or 32j + 16 + 4lg + e - 4 (e >= 4),
  // the order in which the S^T tiles 2j, 2j + 1 deliver the probabilities.
  auto tr_v = [&](Frag (&vt)[4][KS]) __attribute__((always_inline)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int j = 0; j < KS; ++j) {
        const IO* p0 = myV + tr_offset(32 * j + 4 * lg, 16 * dt, D, lr);
        if (32 * j + 16 < kFpRows) {
          vt[dt][j] = C::tr(p0, p0 + 16 * D);
        } else {
          const s16x4 a = lds_tr4(p0);
          const s16x8 c = __builtin_shufflevector(a, s16x4{0, 0, 0, 0}, 0, 1, 2, 3, 4, 5, 6, 7);
          __builtin_memcpy(&vt[dt][j], &c, 16);
        }
        vt[dt][j].v = in_agpr(vt[dt][j].v);
      }
    // every transposed read has returned before the next plane's V lands
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  };
  // K rows of a plane (raw), rows >= N read as zeros
  auto load_k = [&](const __amdgpu_buffer_rsrc_t& rK, Raw8<IO> (&kr)[KT][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < KT; ++u) {
      unsigned v, so;
      tile_off(koff, u, p.sk[2], v, so);
#pragma unroll
      for (int s = 0; s < 2; ++s) kr[u][s] = buf_load8<IO>(rK, v + 64 * s, so);
    }
  };
  // K-hat = R K * scale * log2(e), rounded once (the same staging as the
  // other forward / backward kernels, so every pass sees the same logits)
  auto stage_k = [&](const Raw8<IO> (&kr)[KT][2], Frag (&kf)[KT][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < KT; ++u) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float x[8], cs[8];
        unpack8(kr[u][s], x);
        tab8(u, s, cs);
        rope_rotate8(x, cs);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= c2;
        kf[u][s] = C::make(x);
        kf[u][s].v = in_agpr(kf[u][s].v);
      }
    }
  };

  // Planes of this wave: plane, plane + stride, ...  The next plane's V goes
  // to LDS during subtiles 0 .. 8 of the current one (a few instructions per
  // subtile, so that no wait of the current plane's loads queues behind a
  // whole plane of them), its K rows are loaded during the last subtile (when
  // the K-hat registers are free) and staged with its V^T after the last
  // O product.  A wave without a next plane loads through empty ranges.
  int plane = block_id() * kFpW + wave;
  const int stride = p.n_wg * kFpW;
  if (plane >= planes) return;   // (wave-uniform; no barrier follows)
  Frag vt[4][KS], kf[KT][2];
  Frag ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) C::set(ones, e, 1.f);
  ones.v = in_agpr(ones.v);
  Raw8<IO> qr[KT][2], kr[KT][2];
  // Q rows of subtiles t + 2 .. t + kQpf - 1 are in flight while subtile t runs
  constexpr int kQpf = 5;
  {
    dma_v(plane);
    load_k(rsrc(p.k, p.sk, plane), kr);
    const auto rQ = rsrc(p.q, p.sq, plane);
#pragma unroll
    for (int t = 0; t < kQpf; ++t) load_q(rQ, t, qr[t]);
    tr_v(vt);
    stage_k(kr, kf);
  }
  constexpr int kDmaPer = 3;   // V rows (8 per instruction) of the next plane per subtile
  for (;;) {
    const int nxt = plane + stride;
    const bool more = nxt < planes;
    const int pn = more ? nxt : plane;
    const auto rQ = rsrc(p.q, p.sq, plane);
    const auto rVn = make_rsrc(plane_ptr(p.v, p.sv, pn), more ? (unsigned)(((int64_t)(N - 1) * p.sv[2] + D) * ES) : 0u);
    const auto rKn = make_rsrc(plane_ptr(p.k, p.sk, pn), more ? (unsigned)(((int64_t)(N - 1) * p.sk[2] + D) * ES) : 0u);
    const auto rQn = make_rsrc(plane_ptr(p.q, p.sq, pn), more ? (unsigned)(((int64_t)(N - 1) * p.sq[2] + D) * ES) : 0u);
    const auto rO = make_rsrc(plane_ptr(p.o, p.so, plane), (unsigned)(((int64_t)(N - 1) * p.so[2] + D) * ES));
    const auto rL = make_rsrc(p.lse + (int64_t)plane * N, (unsigned)N * 4u);

    // The 13 tiles' first halves, then their second halves: a product's
    // accumulator input comes from 13 products earlier, never from the one
    // just issued (which would stall the MFMA pipe for the full latency).
    auto logits = [&](const Frag (&q)[2], f32x4 (&s)[KT]) __attribute__((always_inline)) {
#pragma unroll
      for (int u = 0; u < KT; ++u) s[u] = C::mma(kf[u][0], q[0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int u = 0; u < KT; ++u) s[u] = C::mma(kf[u][1], q[1], s[u]);
    };

    // softmax of one subtile (query 16t + lr; this lane's keys 16u + 4lg + i):
    // probabilities as B-operand fragments of O^T += V^T P^T (k-slot e of
    // step j: tile 2j, i = e for e < 4; tile 2j + 1, i = e - 4 otherwise),
    // row max m and row sum l
    auto softmax = [&](f32x4 (&sc)[KT], Frag (&pf)[KS], float& m) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i >= klim) sc[KT - 1][i] = -__builtin_inff();
      float m0 = fmaxf(sc[0][0], sc[0][1]), m1 = fmaxf(sc[0][2], sc[0][3]);
#pragma unroll
      for (int u = 1; u < KT; ++u) {
        m0 = fmaxf(m0, fmaxf(sc[u][0], sc[u][1]));
        m1 = fmaxf(m1, fmaxf(sc[u][2], sc[u][3]));
      }
      m = group4_max(fmaxf(m0, m1));
#pragma unroll
      for (int u = 0; u < KT; ++u) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) e[i] = fast_exp2(sc[u][i] - m);
        C::set2(pf[u >> 1], 2 * (u & 1), e[0], e[1]);
        C::set2(pf[u >> 1], 2 * (u & 1) + 1, e[2], e[3]);
      }
      if constexpr (KT & 1) {
        C::set2(pf[KS - 1], 2, 0.f, 0.f);
        C::set2(pf[KS - 1], 3, 0.f, 0.f);
      }
    };
    // five independent accumulators in turn (each accumulates every 5th
    // product): O^T's four channel tiles and, from an all-ones A operand, the
    // row sum l = sum_k P (the sum of the same rounded probabilities the O
    // product weights V with, so O's weights sum to 1 exactly; every lane
    // receives its query's sum)
    auto pv = [&](const Frag (&pf)[KS], f32x4 (&o)[5]) __attribute__((always_inline)) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] = C::mma(vt[dt][0], pf[0], f32x4{0.f, 0.f, 0.f, 0.f});
      o[4] = C::mma(ones, pf[0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
      for (int j = 1; j < KS; ++j) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = C::mma(vt[dt][j], pf[j], o[dt]);
        o[4] = C::mma(ones, pf[j], o[4]);
      }
    };
    // O rows: lane (lr, lg) holds O[16t + lr][16dt + 4lg + i] (times l)
    auto store_o = [&](int t, const f32x4 (&o)[5], float m) __attribute__((always_inline)) {
      const float l = o[4][0];
      const float inv = __builtin_amdgcn_rcpf(l);
      unsigned ov, os;
      tile_off(ooff, t, p.so[2], ov, os);
#pragma unroll
      for (int d0 = 0; d0 < 4; d0 += 2) {
        unsigned w2[2][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          typedef IO io2 __attribute__((ext_vector_type(2)));
          typedef float f2 __attribute__((ext_vector_type(2)));
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const io2 v = __builtin_convertvector(f2{o[d0 + h][2 * k] * inv, o[d0 + h][2 * k + 1] * inv}, io2);
            w2[h][k] = __builtin_bit_cast(unsigned, v);
          }
        }
        u32x4 w;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto r = __builtin_amdgcn_permlane16_swap(w2[0][k], w2[1][k], false, false);
          w[k] = r[0];
          w[2 + k] = r[1];
        }
        buf_store16(w, rO, ov + 32u * d0, os);
      }
      // LSE of row 16t + lr from lane group 0 (the others address past row
      // N - 1: outside the range)
      const float lse = (m + fast_log2(l)) * kLn2;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse), rL, loff + 64u * t, 0u, 0);
    };

    // Three subtiles in flight: step t issues the logits of subtile t + 1 and
    // the O product of subtile t - 1 on the MFMA pipe while the VALU computes
    // the probabilities of subtile t; one MFMA is scheduled after every few
    // VALU instructions, so that neither waits for the other.
    // Q-hat of subtile t + 1 (qf[(t + 1) & 1]) feeds the logits of step t
    // while that step's VALU already rotates subtile t + 2 into the other buffer
    Frag qf[2][2];
    f32x4 sc[KT], sn[KT], o[5];
    Frag pc[KS], pp[KS];
    float mc = 0.f, mp = 0.f;
    rot_q(qr[0], 0, qf[0]);
    logits(qf[0], sn);
    rot_q(qr[1], 1, qf[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t <= KT; ++t) {
      if (t < KT) {
#pragma unroll
        for (int u = 0; u < KT; ++u) sc[u] = sn[u];
      }
      if (t + 1 < KT) logits(qf[(t + 1) & 1], sn);
      if (t + 2 < KT) rot_q(qr[t + 2], t + 2, qf[t & 1]);
      if (t >= 1) pv(pp, o);
      if (t < KT) softmax(sc, pc, mc);
      const int nm = (t + 1 < KT ? 2 * KT : 0) + (t >= 1 ? 5 * KS : 0);
#pragma unroll
      for (int i = 0; i < 2 * KT + 5 * KS; ++i) {
        if (i < nm) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // four VALU
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // loads before stores: a later wait for one of these loads (the
      // vector memory counter is in order) then does not include the stores
      if (t + kQpf < KT) load_q(rQ, t + kQpf, qr[t + kQpf]);
      if (t == KT - 2) load_k(rKn, kr);   // K-hat's last use (logits of subtile KT-1) is issued
      if (t == KT - 1) {
#pragma unroll
        for (int u = 0; u < kQpf; ++u) load_q(rQn, u, qr[u]);
      }
#pragma unroll
      for (int i = kDmaPer * t; i < kDmaPer * (t + 1); ++i)
        if (i < kFpRows / 8) dma_row8(rVn, i);
      if (t >= 1) store_o(t - 1, o, mp);
      if (t < KT) {
#pragma unroll
        for (int j = 0; j < KS; ++j) pp[j] = pc[j];
        mp = mc;
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!more) break;
    plane = nxt;
    tr_v(vt);
    stage_k(kr, kf);
  }
}

hipError_t launch_fwd_plane(const FwdParams& p0, int io, hipStream_t st) {
  FwdParams p = p0;
  const void* kern = io == DT_F16 ? reinterpret_cast<const void*>(fwd_plane_kernel<f16>)
                                  : reinterpret_cast<const void*>(fwd_plane_kernel<bf16>);
  const int planes = p.B * p.H;
  const int grid = persistent_grid(kern, kFpW * 64, (planes + kFpW - 1) / kFpW);
  if (grid <= 0) return hipErrorInvalidConfiguration;
  p.n_wg = grid;
  if (io == DT_F16)
    hipLaunchKernelGGL(fwd_plane_kernel<f16>, dim3(grid), dim3(kFpW * 64), 0, st, p);
  else
    hipLaunchKernelGGL(fwd_plane_kernel<bf16>, dim3(grid), dim3(kFpW * 64), 0, st, p);
  return hipGetLastError();
}

}  // namespace farope
