// One-pass backward for planes that fit on chip (N <= 256, D = 64).
//
// Reference behaviour followed ("fa_rope_full .py"): delta = rowsum(dO * O)
// (FA:325-357); per key tile P = exp(S - LSE), dV += P^T dO,
// dS = P * (dP - delta), dK-hat += dS^T Q-hat, dK = R^T dK-hat * scale
// (FA:374-691); per query tile dQ-hat += dS K-hat, dQ = R^T dQ-hat * scale
// (FA:708-1009); the CLS row bypasses the rotation (FA:647-662, FA:980-993).
// The reference recomputes S, P and dP in two kernels; here one workgroup
// owns a whole (b, h) plane and computes them once.
//
// Workgroup = 8 waves.  Wave w owns keys 32w .. 32w+31 (two 16-key
// subtiles): their K-hat and V rows sit in registers as MFMA B-operands and
// their dK-hat / dV accumulators in registers.  The rotated K-hat rows of the
// whole plane also stay in LDS (row-major), from which the K-hat^T operand of
// dQ-hat^T = K-hat^T dS^T is read transposed.  The plane's queries are swept in
// stages of 32 rows, double-buffered in LDS, one barrier per stage:
//   commit   staged registers -> LDS: Q-hat and dO rows (row-major),
//            -LSE*log2(e), -delta = -rowsum(dO*O)
//   barrier
//   prefetch next stage's Q, dO, O rows (+ RoPE table rows, LSE)
//   dQ of the previous stage: dQ-hat^T = K-hat^T dS^T from the resident
//            K-hat tile and the key-major dS^T tile that stage left in LDS;
//            un-rotate, store
//   sweep    S and dP for the wave's keys (A = Q-hat / dO rows), P and dS,
//            dS^T -> LDS (key-major, 8-byte writes), dV^T += dO^T P and
//            dK-hat^T += Q-hat^T dS with dO^T / Q-hat^T read transposed
//            straight from the row-major tiles (ds_read_b64_tr_b16)
// Query rows of a 32-row block are used in natural order: for the 16-row
// half h, MFMA output row 4lg+i is query 16h+4lg+i, which is exactly the
// k-slot 4h+i that the transposed reads (rows 16h+4lg+e) deliver.
// Q, K, V, O, dO are read from HBM once; dQ, dK, dV written once.
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

namespace {
constexpr int kPlaneNW = 8;                   // waves per workgroup
constexpr int kPlaneQS = 32;                  // query rows per stage
constexpr int kPlaneMaxN = kPlaneNW * 32;     // keys per workgroup
constexpr int kPlaneLD = 64;                  // pitch of the Q-hat / dO / K-hat tiles (elements)
constexpr int kPlaneLDD = kPlaneQS;           // pitch of the key-major dS^T tile (elements)
}  // namespace

// Unpadded LDS tiles with their 16-byte chunks XOR-swizzled per row.  The
// swizzles are chosen (and checked against a 64-bank model) so that every
// access pattern of the kernel is conflict-free: 16-byte reads of 16
// consecutive rows, transposed 8-byte reads of rows {4lg + e} and
// {8lg + e, 8lg + 4 + e}, 16-byte row writes and 8-byte dS^T writes.  Both
// have period 16 in the row, so row offsets by multiples of 16 stay
// compile-time constants.
// Q-hat / dO / K-hat: 128-byte rows (8 chunks).
__device__ __forceinline__ int sw64(int r, int col) {
  const int f = ((((r >> 1) & 3) ^ ((r >> 2) & 2)) << 1) | ((r >> 3) & 1);
  return r * 64 + ((((col >> 3) ^ f)) << 3) + (col & 7);
}
// dS^T: 64-byte rows (4 chunks).
__device__ __forceinline__ int sw32(int r, int col) {
  return r * 32 + ((((col >> 3) ^ ((r >> 2) & 3))) << 3) + (col & 7);
}

// LDS copy of the RoPE table rows a plane uses, one 256-byte row (32 pairs of
// (cos, sin)) per token.  The sixteen 16-byte chunks of token row r are
// stored in chunk order c ^ (r & 15): sixteen lanes reading the same chunk of
// sixteen consecutive rows, and eight lanes reading a whole row next to eight
// reading the following row, both touch every bank once.
__device__ __forceinline__ f32x4 tab_chunk(const float* t, int row, int c) {
  return *reinterpret_cast<const f32x4*>(t + ((row << 4) + (c ^ (row & 15))) * 4);
}

// VEC: every tensor of the call allows 16-byte vector access (decided on the
// host); the generic instantiation gathers element by element instead.
// NKB: 32-key blocks summed by the dQ products, 8, 7 (for N = 193 .. 224, the
// ViT-S/B planes) or 1 (N <= 32); dS^T rows and K-hat rows of keys >= N are
// zero, so blocks beyond the plane's keys add nothing.
// XD (N <= 32, every key of the plane in wave 0): delta = sum_k P dP, formed
// from the sweep's own fp32 P and dP by a 16-lane sum, instead of
// rowsum(dO * O) from the bf16-stored O.  Both are delta = dO . O exactly;
// with a handful of keys dP - delta is a small difference of near-equal
// terms, and the rounding of the stored O then dominates dS.
template <typename IO, int CT, bool VEC, int NKB, bool XD>
__global__ void __launch_bounds__(kPlaneNW * 64)
bwd_plane_kernel(const BwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  constexpr int LD = kPlaneLD, LDD = kPlaneLDD, QS = kPlaneQS;
  static_assert(sizeof(S) == 2, "the plane kernel stores 16-bit operands");

  __shared__ __attribute__((aligned(16))) S sQ[2][QS * LD];           // Q-hat rows of a stage
  __shared__ __attribute__((aligned(16))) S sG[2][QS * LD];           // dO rows of a stage
  __shared__ __attribute__((aligned(16))) S sdS[2][kPlaneMaxN * LDD]; // dS^T [key][query]
  __shared__ __attribute__((aligned(16))) S sK[kPlaneMaxN * LD];      // K-hat rows of the plane
  __shared__ __attribute__((aligned(16))) float sL2[2][QS];
  __shared__ __attribute__((aligned(16))) float sDl[2][QS];
  extern __shared__ __attribute__((aligned(16))) float sTab[];        // N rows x 64 floats

  const int N = p.N;
  const int planes = p.B * p.H;
  const bool vec_q = VEC || p.vec_q, vec_k = VEC || p.vec_k, vec_v = VEC || p.vec_v;
  const bool vec_o = VEC || p.vec_o, vec_do = VEC || p.vec_do, vec_dq = VEC || p.vec_dq;
  const bool vec_dk = VEC || p.vec_dk, vec_dv = VEC || p.vec_dv;
  const float c2 = p.scale_log2;

  const int tid = thread_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int nkv32 = round_up32(N);
  const int nstages = (N + QS - 1) / QS;
  const int kw = 32 * wave;                                    // first key of this wave
  const int nu = (kw < N) + (kw + 16 < N);                     // active 16-key subtiles
  const int dd = wave & 3;    // head-dim slice 16dd .. 16dd+15 of this wave's dQ tile
  const int qt = wave >> 2;   // and its 16-query subtile of a stage

  // Persistent: workgroup g handles planes g, g + G, g + 2G, ... (G = grid),
  // dealt XCD-major so that consecutive planes of an XCD share its L2.
  const int pos = xcd_remap(block_id(), p.n_wg);
  auto item_of = [&](int it) {
    const int item = it * p.n_wg + pos;
    return item < planes ? item : -1;
  };
  // (plane is wave-uniform; readfirstlane keeps the address arithmetic and
  // the descriptors built from it in SGPRs even where the compiler would
  // otherwise carry the value through a divergent branch in VGPRs)
  auto base = [&](const void* b, const int64_t* st, int plane_) {
    const int plane = __builtin_amdgcn_readfirstlane(plane_);
    const int bb = plane / p.H, hh = plane - bb * p.H;
    return static_cast<const IO*>(b) + bb * st[0] + hh * st[1];
  };
  // VEC: the host guarantees unit d-stride, 16-byte alignment and in-plane
  // byte offsets below 2^31.  Tensors are then read and written through
  // buffer descriptors over rows 0 .. N-1 of the plane (SGPRs), with 32-bit
  // lane byte offsets fixed for the whole kernel and uniform per-stage
  // offsets: no 64-bit address arithmetic per lane, and rows >= N read as 0.
  // Otherwise: generic strided 64-bit addressing.
  constexpr unsigned ES = sizeof(IO);
  auto rsrc = [&](const void* b, const int64_t* st, int plane) {
    return make_rsrc(base(b, st, plane), (unsigned)(((int64_t)(N - 1) * st[2] + 64) * ES));
  };
  auto boff = [&](const int64_t* st, int row, int col) {   // lane byte offset (VEC)
    return (unsigned)((row * (int)st[2] + col) * (int)ES);
  };

  // ---- stage staging: thread t < 256 carries row t/8, channels 8*(t%8) .. +7
  //      of Q, dO and O; threads 256 .. 256+QS-1 carry the stage's LSE ----
  Raw8<IO> pq, pg, po;
  float plse = 0.f;
  const int ssr = (tid >> 3) & 31, ssc = tid & 7;   // staging row / chunk of this thread
  unsigned bq = 0, bg = 0, bo = 0;
  if constexpr (VEC) {
    bq = boff(p.sq, ssr, 8 * ssc);
    bg = boff(p.sdo, ssr, 8 * ssc);
    bo = boff(p.so, ssr, 8 * ssc);
  }
  // Buffer descriptors of the staged rows of one plane (SGPRs).  They are
  // built once per plane, in the last stage of the previous plane, whose
  // prefetch is the first to read the plane, instead of per stage (the (b, h)
  // split of the plane index and the 64-bit base arithmetic are most of a
  // stage's scalar work).
  struct StageRs {
    __amdgpu_buffer_rsrc_t q, g, o, l;
  };
  auto stage_rs = [&](int plane) __attribute__((always_inline)) {
    return StageRs{rsrc(p.q, p.sq, plane), rsrc(p.dout, p.sdo, plane), rsrc(p.o, p.so, plane),
                   make_rsrc(p.lse + (int64_t)plane * N, (unsigned)N * 4u)};
  };
  auto prefetch = [&](int plane, const StageRs& rs, int qb) __attribute__((always_inline)) {
    if constexpr (VEC) {
      if (tid < 256) {   // waves 0..3 (wave-uniform)
        pq = buf_load8<IO>(rs.q, bq, (unsigned)(qb * (int)p.sq[2] * (int)ES));
        pg = buf_load8<IO>(rs.g, bg, (unsigned)(qb * (int)p.sdo[2] * (int)ES));
        po = buf_load8<IO>(rs.o, bo, (unsigned)(qb * (int)p.so[2] * (int)ES));
      }
    } else {
      const int t = opaque(tid), sr = (t >> 3) & 31, sc = t & 7, gr = qb + sr;
      if (t < 256 && gr < N) {
        pq = load_raw8(base(p.q, p.sq, plane) + gr * p.sq[2] + 8 * sc * p.sq[3], p.sq[3], vec_q);
        pg = load_raw8(base(p.dout, p.sdo, plane) + gr * p.sdo[2] + 8 * sc * p.sdo[3], p.sdo[3], vec_do);
        po = load_raw8(base(p.o, p.so, plane) + gr * p.so[2] + 8 * sc * p.so[3], p.so[3], vec_o);
      } else {
        pq = pg = po = zero_raw8<IO>();
      }
    }
    // raw LSE (scaled and masked at commit, so no wait is forced here: a
    // wait on this load would also drain the Q / dO / O loads issued above);
    // the buffer range is the plane's N values, rows >= N read 0
    const int lt = tid - 256;
    if (lt >= 0 && lt < QS)
      plse = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs.l, (unsigned)lt * 4u, (unsigned)qb * 4u, 0));
  };
  auto commit = [&](int buf, int qb) __attribute__((always_inline)) {
    const int t = tid, sr = ssr, sc = ssc;
    if (t < 256) {
      float x[8], g[8];
      unpack8(pq, x);
      // Q-hat = R q (rows >= N are zero either way)
      const int row = min(qb + sr, N - 1);
      const f32x4 c0 = tab_chunk(sTab, row, 2 * sc), c1 = tab_chunk(sTab, row, 2 * sc + 1);
      const float cs[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
      rope_rotate8(x, cs);
      C::put8(&sQ[buf][sw64(sr, 8 * sc)], x);
      if constexpr (std::is_same<IO, S>::value) {
        *reinterpret_cast<typename Raw8<IO>::vec*>(&sG[buf][sw64(sr, 8 * sc)]) = pg.v;   // raw dO row segment
      } else {
        unpack8(pg, g);
        C::put8(&sG[buf][sw64(sr, 8 * sc)], g);
      }
      // delta = rowsum(dO * O); the 8 chunks of a row are 8 consecutive lanes
      const float d = dpp_sum8(dot8(pg, po, 0.f));
      if (sc == 0) sDl[buf][sr] = -d;   // stored negated: it seeds the dP accumulators
    } else if (t - 256 < QS) {
      // -LSE in log2 units seeds the logit accumulators (rows >= N: -inf, so P = 0)
      sL2[buf][t - 256] = qb + (t - 256) < N ? -plse * kLog2e : -INFINITY;
    }
  };

  // ---- own keys kw + 16u + lr: raw K / V row segments in flight ----
  Raw8<IO> rk[2][2], rv[2][2];
  // VEC lane byte offsets: K / V at (row kw + 16u + lr, channel 8lg); dK / dV
  // at (row kw + 16u + lr, channel 4lg)
  unsigned bk[2] = {0, 0}, bv[2] = {0, 0}, bdk[2] = {0, 0}, bdv[2] = {0, 0};
  if constexpr (VEC) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      bk[u] = boff(p.sk, kw + 16 * u + lr, 8 * lg);
      bv[u] = boff(p.sv, kw + 16 * u + lr, 8 * lg);
      bdk[u] = boff(p.sdk, kw + 16 * u + lr, 4 * lg);
      bdv[u] = boff(p.sdv, kw + 16 * u + lr, 4 * lg);
    }
  }
  auto prefetch_kv = [&](int plane) __attribute__((always_inline)) {
    if constexpr (VEC) {
      const auto rK = rsrc(p.k, p.sk, plane), rV = rsrc(p.v, p.sv, plane);
#pragma unroll
      for (int u = 0; u < 2; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          rk[u][s] = buf_load8<IO>(rK, bk[u], 32 * s * ES);
          rv[u][s] = buf_load8<IO>(rV, bv[u], 32 * s * ES);
        }
    } else {
      const int lane = opaque(tid & 63), lr = lane & 15, lg = lane >> 4;
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = kw + 16 * u + lr;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int c0 = 32 * s + 8 * lg;
          if (row < N) {
            rk[u][s] = load_raw8(base(p.k, p.sk, plane) + row * p.sk[2] + c0 * p.sk[3], p.sk[3], vec_k);
            rv[u][s] = load_raw8(base(p.v, p.sv, plane) + row * p.sv[2] + c0 * p.sv[3], p.sv[3], vec_v);
          } else {
            rk[u][s] = rv[u][s] = zero_raw8<IO>();
          }
        }
      }
    }
  };
  // K-hat and V rows as B-operands; K-hat rows also go to sK (all 256 rows, zero beyond N)
  Frag kf[2][2], vf[2][2];
  auto commit_kv = [&]() __attribute__((always_inline)) {
    const int lane = opaque(tid & 63), lr = lane & 15, lg = lane >> 4;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = min(kw + 16 * u + lr, N - 1);
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float x[8], y[8];
        const f32x4 t0 = tab_chunk(sTab, row, 8 * s + 2 * lg), t1 = tab_chunk(sTab, row, 8 * s + 2 * lg + 1);
        const float cs[8] = {t0[0], t0[1], t0[2], t0[3], t1[0], t1[1], t1[2], t1[3]};
        unpack8(rk[u][s], x);
        unpack8(rv[u][s], y);
        rope_rotate8(x, cs);
        // K-hat pre-scaled by softmax_scale * log2(e): the logits product then
        // yields S in log2 units directly (dQ's scale divides it out again)
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= c2;
        kf[u][s] = C::make(x);
        vf[u][s] = C::make(y);
        // materialise V here (for 16-bit I/O the conversion folds away and the
        // fragment would alias the load registers, moving the wait for these
        // loads into the first sweep, behind the next stage's prefetch)
        asm volatile("" : "+v"(vf[u][s].v));
        *reinterpret_cast<decltype(kf[u][s].v)*>(&sK[sw64(kw + 16 * u + lr, 32 * s + 8 * lg)]) =
            kf[u][s].v;
      }
    }
  };

  // dQ-hat = dS K-hat * scale with K-hat stored pre-scaled by c2
  const float dq_scale = p.scale / c2;

  f32x4 dvacc[2][4], dkacc[2][4];

  // A-operands of this wave's dQ tile, K-hat^T rows 16dd .. 16dd+15 of every
  // 32-key block (k = keys 32kb + 8lg + (0..7)), read transposed from sK.
  // Lane parts of the read offsets are rows 8lg + lr/4 and 8lg + 4 + lr/4,
  // column 4(lr%4) of the slice; the key block adds a compile-time constant
  // (the swizzles have period 16 in the row).  Rows of keys >= N are zero.
  // With 16-bit I/O they are read once per plane and kept in registers for
  // all of its stages; 32-bit I/O needs those registers for its staging and
  // reads them per stage.
  constexpr bool KQREG = sizeof(IO) == 2;
  Frag kq[KQREG ? NKB : 1];
  auto ka_tr = [&](int kb) __attribute__((always_inline)) {
    const int lane = opaque(tid & 63), lr = lane & 15, lg = lane >> 4;
    const int r0 = 8 * lg + (lr >> 2);
    const S* ka0 = &sK[sw64(r0, 16 * dd + 4 * (lr & 3))];
    const S* ka1 = &sK[sw64(r0 + 4, 16 * dd + 4 * (lr & 3))];
    return C::tr(ka0 + 32 * kb * LD, ka1 + 32 * kb * LD);
  };
  auto load_kq = [&]() __attribute__((always_inline)) {
    if constexpr (KQREG) {
      // the two lane addresses once for all blocks (ka_tr would form them
      // again per block from its opaque lane copy)
      const int lane = opaque(tid & 63), lr = lane & 15, lg = lane >> 4;
      const int r0 = 8 * lg + (lr >> 2);
      const S* ka0 = &sK[sw64(r0, 16 * dd + 4 * (lr & 3))];
      const S* ka1 = &sK[sw64(r0 + 4, 16 * dd + 4 * (lr & 3))];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) kq[kb] = C::tr(ka0 + 32 * kb * LD, ka1 + 32 * kb * LD);
    }
  };

  // ---- dQ of one finished stage from its dS^T tile: this wave's 16x16 tile
  //      dQ-hat^T[16dd.., 16qt..] = K-hat^T dS^T, un-rotated and stored.
  //      NKB = number of 32-key blocks (straight-line code, no per-block branch) ----
  // VEC lane byte offset of this lane's dQ element (row 16qt + lr of a stage, channel 16dd + 4lg)
  const unsigned bdq = VEC ? boff(p.sdq, 16 * qt + lr, 16 * dd + 4 * lg) : 0u;
  // lane parts of the transposed dS^T read offsets (as for kq), kept for the
  // whole kernel: per stage only the buffer base changes
  const int dqr0 = 8 * lg + (lr >> 2);
  const int dqo0 = sw32(dqr0, 16 * qt + 4 * (lr & 3)), dqo1 = sw32(dqr0 + 4, 16 * qt + 4 * (lr & 3));
  // (buf = sp & 1; a compile-time constant inside the stage loop)
  auto dq = [&](int plane, __amdgpu_buffer_rsrc_t rdq, int sp, int buf) __attribute__((always_inline)) {
    const int qb = sp * QS;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    const S* db0 = &sdS[buf][dqo0];
    const S* db1 = &sdS[buf][dqo1];
    // A = K-hat^T rows 16dd.., B = dS^T columns 16qt..; k = keys 32kb + 8lg + (0..7).
    // The B fragment of block kb+1 is read before the product of block kb,
    // so each product waits for a read issued one product earlier rather
    // than for a full LDS round trip.
    Frag b2[2];
    b2[0] = C::tr(db0, db1);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      if (kb + 1 < NKB) b2[(kb + 1) & 1] = C::tr(db0 + 32 * (kb + 1) * LDD, db1 + 32 * (kb + 1) * LDD);
      if constexpr (KQREG)
        acc = C::mma(kq[kb], b2[kb & 1], acc);
      else
        acc = C::mma(ka_tr(kb), b2[kb & 1], acc);
    }
    const int row = qb + 16 * qt + lr;
    auto unrotate = [&](int trow, float (&g4)[4]) __attribute__((always_inline)) {
      const f32x4 t = tab_chunk(sTab, trow, 4 * dd + lg);   // pairs 8dd + 2lg + (0, 1)
#pragma unroll
      for (int r = 0; r < 2; ++r) {   // g = R^T g-hat
        const float e = acc[2 * r] * dq_scale, o = acc[2 * r + 1] * dq_scale;
        const float c = t[2 * r], sn = t[2 * r + 1];
        g4[2 * r] = e * c + o * sn;
        g4[2 * r + 1] = o * c - e * sn;
      }
    };
    if constexpr (VEC) {
      // unconditional: rows >= N fall outside the descriptor range and are dropped
      float g4[4];
      unrotate(min(row, N - 1), g4);
      buf_store4<IO>(rdq, bdq, (unsigned)(qb * (int)p.sdq[2] * (int)ES), g4);
    } else if (row < N) {
      float g4[4];
      unrotate(row, g4);
      {
        IO* __restrict__ dQ = const_cast<IO*>(base(p.dq, p.sdq, plane));
        store4(dQ + row * p.sdq[2] + (16 * dd + 4 * lg) * p.sdq[3], p.sdq[3], vec_dq, g4);
      }
    }
  };
  // ---- S, dP, P, dS, dV, dK for the wave's two subtiles over one 32-query
  //      stage (query rows in natural order, see above).  Keys >= N (the rest
  //      of the subtile holding key N-1, and all of a subtile past it) need no
  //      mask: their K-hat and V rows are zero, so S = dP = 0 there and P, dS
  //      are finite (P is clamped to [0, 1], which the exact P never leaves);
  //      their dS^T rows meet zero K-hat rows in the dQ products and their dK /
  //      dV rows are never stored.  One code path for every active wave keeps the
  //      dK / dV accumulators in the same registers across stages (a per-wave
  //      choice between sweep variants makes the compiler copy all of them at
  //      the join every stage), and a wave with one live subtile shares its
  //      SIMD with a fully loaded one anyway. ----
  // live1: some query of the stage's second 16-row half is below N.  When
  // none is (the last stage of N = 193 .. 208, ViT-S/B), that half's S / dP
  // products and probabilities are skipped: its P and dS fragment slots are
  // zero for the dV / dK products, and its dS^T columns are left as they are,
  // because they only reach dQ rows >= N, which are never stored.
  // F0 (a std::bool_constant): the plane's first stage, whose dV / dK
  // products start from zero accumulators instead of adding to them.
  auto sweep_keys = [&](int buf, bool live1, auto f0c) __attribute__((always_inline)) {
    constexpr int NUA = 2;
    constexpr bool F0 = decltype(f0c)::value;
    const S* q = &sQ[buf][0];
    const S* g = &sG[buf][0];
    S* ds = &sdS[buf][0];
    {
      Frag pf[NUA], dsf[NUA];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 1 && !live1) {
#pragma unroll
          for (int u = 0; u < NUA; ++u) {
            C::set2(pf[u], 2, 0.f, 0.f);
            C::set2(pf[u], 3, 0.f, 0.f);
            C::set2(dsf[u], 2, 0.f, 0.f);
            C::set2(dsf[u], 3, 0.f, 0.f);
          }
          continue;
        }
        const int q0 = 16 * h + 4 * lg;   // queries q0 .. q0+3 in this lane
        const f32x4 nl2 = *reinterpret_cast<const f32x4*>(&sL2[buf][q0]);   // -LSE * log2(e)
        const f32x4 ndl = *reinterpret_cast<const f32x4*>(&sDl[buf][q0]);   // -delta
        // accumulators start at -LSE (S, in log2 units through the pre-scaled
        // K-hat) and at -delta (dP): P = exp2(acc) and dP - delta need no
        // further arithmetic
        f32x4 sacc[NUA], pacc[NUA];
#pragma unroll
        for (int u = 0; u < NUA; ++u) {
          sacc[u] = nl2;
          pacc[u] = XD ? f32x4{0.f, 0.f, 0.f, 0.f} : ndl;
        }
        const int qr = 16 * h + lr;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const Frag a = C::lds(q + sw64(qr, 32 * s + 8 * lg));
          const Frag b = C::lds(g + sw64(qr, 32 * s + 8 * lg));
#pragma unroll
          for (int u = 0; u < NUA; ++u) {
            sacc[u] = C::mma(a, kf[u][s], sacc[u]);
            pacc[u] = C::mma(b, vf[u][s], pacc[u]);
          }
        }
        // XD: delta of queries q0 + i = sum over the wave's 32 keys (lanes lr,
        // subtiles u) of P dP; keys >= N have dP = 0, queries >= N P = 0
        float xdl[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (XD) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float t = 0.f;
#pragma unroll
            for (int u = 0; u < NUA; ++u)
              t = __builtin_fmaf(__builtin_amdgcn_fmed3f(fast_exp2(sacc[u][i]), 0.f, 1.f), pacc[u][i], t);
            t = dpp_sum8(t);
            xdl[i] = t + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(t), 0x140, 0xF, 0xF, false));   // row_mirror
          }
        }
#pragma unroll
        for (int u = 0; u < NUA; ++u) {
          float pv[4], dsv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) pv[i] = __builtin_amdgcn_fmed3f(fast_exp2(sacc[u][i]), 0.f, 1.f);
#pragma unroll
          for (int i = 0; i < 4; ++i) dsv[i] = pv[i] * (XD ? pacc[u][i] - xdl[i] : pacc[u][i]);
          C::set2(pf[u], 2 * h, pv[0], pv[1]);
          C::set2(pf[u], 2 * h + 1, pv[2], pv[3]);
          C::set2(dsf[u], 2 * h, dsv[0], dsv[1]);
          C::set2(dsf[u], 2 * h + 1, dsv[2], dsv[3]);
          C::put4(ds + sw32(kw + 16 * u + lr, q0), dsf[u], h);
        }
      }
      // dV^T += dO^T P ; dK-hat^T += Q-hat^T dS  (k = queries 16h + 4lg + e)
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const int o0 = sw64(4 * lg + (lr >> 2), 16 * d + 4 * (lr & 3));   // rows 4lg + e
        const int o1 = o0 + 16 * LD;                                      // rows 16 + 4lg + e
        const Frag ag = C::tr(g + o0, g + o1);
        const Frag aq = C::tr(q + o0, q + o1);
#pragma unroll
        for (int u = 0; u < NUA; ++u) {
          dvacc[u][d] = C::mma(ag, pf[u], F0 ? f32x4{0.f, 0.f, 0.f, 0.f} : dvacc[u][d]);
          dkacc[u][d] = C::mma(aq, dsf[u], F0 ? f32x4{0.f, 0.f, 0.f, 0.f} : dkacc[u][d]);
        }
      }
    }
  };

  int it = 0;
  int plane = item_of(0);
  if (plane < 0) return;
  StageRs rs = stage_rs(plane);
  prefetch(plane, rs, 0);
  prefetch_kv(plane);
  {
    // table rows shift .. N-1+shift of the packed table -> sTab (token order, swizzled)
    const int shift = 1 - p.has_cls;
    const f32x4* src = reinterpret_cast<const f32x4*>(p.rope) + shift * 16;
    // all of a thread's loads first, then its LDS writes: one memory round
    // trip instead of one per row group (N <= 256 rows: at most 8 per thread)
    constexpr int TIT = kPlaneMaxN * 16 / (kPlaneNW * 64);
    f32x4 tv[TIT];
#pragma unroll
    for (int j = 0; j < TIT; ++j) {
      const int i = tid + j * kPlaneNW * 64;
      tv[j] = i < N * 16 ? src[i] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < TIT; ++j) {
      const int i = tid + j * kPlaneNW * 64, r = i >> 4, c = i & 15;
      if (i < N * 16) *reinterpret_cast<f32x4*>(&sTab[((r << 4) + (c ^ (r & 15))) * 4]) = tv[j];
    }
    // dS^T rows of waves with no key < N (keys >= round_up32(N)) enter the
    // dQ products but are never written by a sweep: zero them once, in both
    // buffers.  (Keys >= N of an active wave are written with dS = 0 by its
    // sweep.)
#pragma unroll
    for (int b = 0; b < 2; ++b)
      for (int i = nkv32 * LDD + tid; i < kPlaneMaxN * LDD; i += kPlaneNW * 64) sdS[b][i] = S(0.f);
  }
  // the table copy and the zeroed rows are visible
  lds_barrier();
  // The first stage of every plane sets the dV / dK accumulators of a wave
  // with keys < N; a wave without any keeps whatever they hold (its stores
  // fall past N and are dropped).  Defined once here.
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int d = 0; d < 4; ++d) dvacc[u][d] = dkacc[u][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  while (plane >= 0) {
    const int nxt = item_of(it + 1);
    const auto rdq = rsrc(p.dq, p.sdq, plane);   // (VEC)
    // The previous plane's last reads of sQ / sG / sL2 / sDl (its last sweep)
    // precede its tail barrier, so these writes need no barrier of their own.
    // sK is read by load_kq right after the barrier below (16-bit I/O), or,
    // with 32-bit I/O, by every dQ product including the previous plane's
    // tail dQ; that variant ends each plane with a barrier (see the loop end)
    // so that no wave rewrites its sK rows while another still reads them.
    commit_kv();
    commit(0, 0);
    // sK and the first stage are complete, and every wave has finished the
    // previous plane's dQ tail (which reads sdS) before the first sweep of
    // this plane writes it
    lds_barrier();
    load_kq();

    // One query stage.  The stage loop runs two stages per trip, so the LDS
    // buffer index BUF is a compile-time constant and the buffers' addresses
    // fold into the LDS instructions' offsets.  FIRST: stage 0 (already
    // committed above, no dQ of a previous stage).
    auto stage = [&](int st, auto bufc, auto firstc) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      constexpr bool FIRST = decltype(firstc)::value;
      const int qb = st * QS;
      if constexpr (!FIRST) {
        commit(buf, qb);
        lds_barrier();
      }
      // next stage, or the next plane's first stage (the last plane re-reads its
      // own first stage).  One unconditional call with a uniformly selected
      // target: the loads land directly in the staging registers, with no
      // merge copies that would force an early wait on them.
      {
        const bool last = st + 1 == nstages;
        const int tp = last ? (nxt >= 0 ? nxt : plane) : plane;
        if (last) rs = stage_rs(tp);
        prefetch(tp, rs, last ? 0 : qb + QS);
      }
      if constexpr (!FIRST) dq(plane, rdq, st - 1, buf ^ 1);
      if (nu > 0) sweep_keys(buf, qb + 16 < N, firstc);
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    stage(0, B0{}, std::true_type{});
    int st = 1;
    for (; st + 1 < nstages; st += 2) {
      stage(st, B1{}, std::false_type{});
      stage(st + 1, B0{}, std::false_type{});
    }
    if (st < nstages) stage(st, B1{}, std::false_type{});

    // kf / vf are dead: start the next plane's own K / V rows, then finish this
    // plane: dQ of the last stage, dK / dV
    prefetch_kv(nxt >= 0 ? nxt : plane);
    lds_barrier();
    dq(plane, rdq, nstages - 1, (nstages - 1) & 1);
    // ---- dK / dV epilogue: lane holds dV /
    //      dK-hat of key kw + 16u + lr, channels 16d + 4lg + (0..3) ----
    if constexpr (VEC && sizeof(IO) == 2) {
      // Unconditional 16-byte descriptor stores: keys >= N (all of an
      // inactive subtile) fall outside the range and are dropped.  Lane
      // groups lg and lg^1 trade halves (v_permlane16_swap) so that each lane
      // writes 8 consecutive channels: even lg channels 16d0 + 4lg .. +7, odd
      // lg channels 16(d0+1) + 4(lg-1) .. +7, for d0 = 0, 2.
      const int lane = tid & 63, lr = lane & 15, lg = lane >> 4;
      const auto rdK = rsrc(p.dk, p.sdk, plane), rdV = rsrc(p.dv, p.sdv, plane);
      typedef IO io4 __attribute__((ext_vector_type(4)));
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = kw + 16 * u + lr;
        const int trow = min(row, N - 1);
#pragma unroll
        for (int d0 = 0; d0 < 4; d0 += 2) {
          u32x2 wv[2], wk[2];
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int d = d0 + j;
            io4 a, g;
            const f32x4 t = tab_chunk(sTab, trow, 4 * d + lg);   // pairs 8d + 2lg + (0, 1)
#pragma unroll
            for (int r = 0; r < 2; ++r) {   // g = R^T g-hat
              const float e = dkacc[u][d][2 * r] * p.scale, o = dkacc[u][d][2 * r + 1] * p.scale;
              const float c = t[2 * r], sn = t[2 * r + 1];
              g[2 * r] = (IO)(e * c + o * sn);
              g[2 * r + 1] = (IO)(o * c - e * sn);
              a[2 * r] = (IO)dvacc[u][d][2 * r];
              a[2 * r + 1] = (IO)dvacc[u][d][2 * r + 1];
            }
            __builtin_memcpy(&wv[j], &a, 8);
            __builtin_memcpy(&wk[j], &g, 8);
          }
          u32x4 xv, xk;
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const auto rv = __builtin_amdgcn_permlane16_swap(wv[0][k], wv[1][k], false, false);
            const auto rk = __builtin_amdgcn_permlane16_swap(wk[0][k], wk[1][k], false, false);
            xv[k] = rv[0];
            xv[2 + k] = rv[1];
            xk[k] = rk[0];
            xk[2 + k] = rk[1];
          }
          const int ch = 16 * (d0 + (lg & 1)) + 4 * (lg & 2);
          buf_store16(xv, rdV, boff(p.sdv, row, ch), 0u);
          buf_store16(xk, rdK, boff(p.sdk, row, ch), 0u);
        }
      }
    } else {
      const int lane = VEC ? tid & 63 : opaque(tid & 63), lr = lane & 15, lg = lane >> 4;
      IO* __restrict__ dK = const_cast<IO*>(base(p.dk, p.sdk, plane));
      IO* __restrict__ dV = const_cast<IO*>(base(p.dv, p.sdv, plane));
      const auto rdK = rsrc(p.dk, p.sdk, plane), rdV = rsrc(p.dv, p.sdv, plane);
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int row = kw + 16 * u + lr;
        if (u < nu && row < N) {
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            float v4[4], g4[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v4[r] = dvacc[u][d][r];
            if constexpr (VEC)
              buf_store4<IO>(rdV, bdv[u], 16 * d * ES, v4);
            else
              store4(dV + row * p.sdv[2] + (16 * d + 4 * lg) * p.sdv[3], p.sdv[3], vec_dv, v4);
            const f32x4 t = tab_chunk(sTab, row, 4 * d + lg);   // pairs 8d + 2lg + (0, 1)
#pragma unroll
            for (int r = 0; r < 2; ++r) {   // g = R^T g-hat
              const float e = dkacc[u][d][2 * r] * p.scale, o = dkacc[u][d][2 * r + 1] * p.scale;
              const float c = t[2 * r], sn = t[2 * r + 1];
              g4[2 * r] = e * c + o * sn;
              g4[2 * r + 1] = o * c - e * sn;
            }
            if constexpr (VEC)
              buf_store4<IO>(rdK, bdk[u], 16 * d * ES, g4);
            else
              store4(dK + row * p.sdk[2] + (16 * d + 4 * lg) * p.sdk[3], p.sdk[3], vec_dk, g4);
          }
        }
      }
    }
    // 32-bit I/O reads K-hat^T from sK in the tail dQ above: every wave must
    // be past it before the next plane's commit_kv overwrites sK (the
    // barrier orders LDS only, so the dK / dV stores stay in flight).
    if constexpr (!KQREG) {
      if (nxt >= 0) lds_barrier();   // nxt is workgroup-uniform
    }
    plane = nxt;
    ++it;
  }
}

int bwd_fused_rows() { return kPlaneMaxN; }

template <typename IO, int CT>
static hipError_t fused_launch(const BwdParams& p0, hipStream_t st) {
  BwdParams p = p0;
  const bool vec = p.vec_q && p.vec_k && p.vec_v && p.vec_o && p.vec_do && p.vec_dq && p.vec_dk &&
                   p.vec_dv;
  const bool nkb7 = (p.N + 31) / 32 == 7, small = p.N <= 32;
  auto kern = small ? (vec ? bwd_plane_kernel<IO, CT, true, 1, true> : bwd_plane_kernel<IO, CT, false, 1, true>)
              : vec ? (nkb7 ? bwd_plane_kernel<IO, CT, true, 7, false> : bwd_plane_kernel<IO, CT, true, 8, false>)
                    : bwd_plane_kernel<IO, CT, false, 8, false>;
  const size_t tab_bytes = (size_t)p.N * 64 * sizeof(float);   // LDS copy of the RoPE rows
  const int grid = persistent_grid(reinterpret_cast<const void*>(kern), kPlaneNW * 64, p.B * p.H,
                                   tab_bytes);
  if (grid <= 0) return hipErrorInvalidValue;
  p.n_wg = grid;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kPlaneNW * 64), tab_bytes, st, p);
  return hipGetLastError();
}

template <typename IO>
static hipError_t fused_ct(const BwdParams& p, int ct, hipStream_t st) {
  switch (ct) {
    case DT_BF16: return fused_launch<IO, DT_BF16>(p, st);
    case DT_F16: return fused_launch<IO, DT_F16>(p, st);
    default: return hipErrorInvalidValue;   // fp32 compute uses the split kernels
  }
}

hipError_t launch_bwd_fused(const BwdParams& p, int io, int ct, hipStream_t st) {
  switch (io) {
    case DT_BF16: return fused_ct<bf16>(p, ct, st);
    case DT_F16: return fused_ct<f16>(p, ct, st);
    default: return fused_ct<float>(p, ct, st);
  }
}

}  // namespace farope
