// Key tiles of the split backward with fp16 dS products (bf16 compute,
// head_dim 128, 16-bit I/O, vector access): dK and dV.
//
// Reference behaviour followed ("fa_rope_full .py"): per key tile
// P = exp(S - LSE), dV += P^T dO, dS = P * (dP - delta), dK-hat += dS^T Q-hat,
// dK = R^T dK-hat * scale, the CLS row bypassing the rotation
// (_attn_bwd_dk_dv_rope, FA:374-691; FA:647-662).
//
// Runs after bwd_dq_kernel (or the stored-dS row pass, bwd_ds.hip), which
// writes what this kernel stages per query stage: delta, the fp16 rotated rows
// Q-hat * c2 (c2 = scale * log2 e, its logit operand) and per-row statistics
// {|dO|_2, max |Q-hat c2|}.  DS (the stored-dS backward): the tile also stores
// its fp16 sig dS^T blocks, its K-hat * fk rows and the exponent of
// 1 / (sig fk), the operands of that backward's dQ GEMM.  One 8-wave
// workgroup per (plane, 128-key tile), the layout of the generic dK/dV kernel
// (bwd.hip): each wave's K-hat and V rows are MFMA B operands in registers,
// and the Q-hat / dO rows of each 64-query stage are staged in LDS (rows
// vperm'd, two buffers: the next stage is committed between the current
// stage's two query blocks) and read transposed for the dV / dK products.
//
// Products in fp16.  The logits take fp16 Q-hat * c2 * fq and K-hat * fk as
// in the forward pass; dK-hat takes dS in fp16, scaled by a power of two sig,
// against the same fp16 Q-hat rows: one MFMA instead of the split-bf16 dS pair
// of the generic kernel, and Q-hat keeps 11 significant bits instead of
// bf16's 8 (the rounding of Q-hat as the dK product's operand was the largest
// term of dK's error there).  dP = dO V and dV = P^T dO stay bf16.  The
// scalings are fixed before the first product, from ranges, so no pass is
// ever repeated:
//  * fq, fk: from the plane's max |Q-hat * c2| (row statistics) and the
//    tile's max |K-hat|.  Both inside [2^-10, 2^12): 1 (the dQ kernel's fp16
//    rows serve).  Otherwise f16_fit (common.h) puts each into [2^14, 2^15)
//    and the tile rotates its Q rows itself.
//  * sig: |dS| = P |dP - delta| <= max_q |dO_q|_2 max_k |V_k|_2 + max_q |delta_q|
//    over the plane's queries and the tile's keys; sig = f16_fit of that
//    bound, so sig dS never overflows fp16 and its largest values keep full
//    precision.  sig is folded into the V operand (exact: a power of two) and
//    into the delta seed of the dP accumulators.
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

namespace {
constexpr int kKeysD = 128;

template <typename IO>
__device__ __forceinline__ const IO* plane_ptr(const void* b, const int64_t* st, int plane, int H) {
  const int bb = plane / H, hh = plane - bb * H;
  return static_cast<const IO*>(b) + bb * st[0] + hh * st[1];
}
}  // namespace

// ---------------------------------------------------------------------------
// Key tiles.
// ---------------------------------------------------------------------------
template <typename IO, bool DS>
__global__ void __launch_bounds__(512) bwd_keys_kernel(const BwdParams p) {
  using C = Comp<DT_BF16>;   // dP = dO V and dV = P^T dO
  using H = Comp<DT_F16>;    // logits and dK-hat
  using Frag = C::Frag;
  using HFrag = H::Frag;
  constexpr int D = kKeysD, NW = 8, QS = 64, KS = D / 32, DT = D / 16, D2 = D / 2, CPR = D / 8;
  constexpr int NT = NW * 64, ITER = QS * CPR / NT;
  constexpr int KROWS = NW * 16;
  constexpr int LDQ = D + 8;    // Q-hat / dO row pitch (elements)
  constexpr unsigned ES = sizeof(IO);
  static_assert(KROWS == kKeysRows && sizeof(IO) == 2 && ITER * NT == QS * CPR, "tile shape");

  // stage buffers (two: the next stage is committed during the current one,
  // into the buffer the previous stage read, which every wave finished before
  // the current stage's barrier; one barrier per stage)
  __shared__ __attribute__((aligned(16))) f16 sQf[2][QS * LDQ];    // fp16 Q-hat * c2 * fq (rows vperm'd)
  __shared__ __attribute__((aligned(16))) bf16 sG[2][QS * LDQ];    // dO rows (vperm'd)
  __shared__ __attribute__((aligned(16))) float sL2[2][QS];        // -LSE2 * fq * fk
  __shared__ __attribute__((aligned(16))) float sDl[2][QS];        // -delta * sig
  __shared__ float sRed[NW][6];

  const int N = p.N;
  const int tile = xcd_remap(block_id(), p.n_wg);
  const int plane = tile / p.n_blk;
  const int kblk = tile - plane * p.n_blk;
  const IO* __restrict__ Q = plane_ptr<IO>(p.q, p.sq, plane, p.H);
  const IO* __restrict__ K = plane_ptr<IO>(p.k, p.sk, plane, p.H);
  const IO* __restrict__ V = plane_ptr<IO>(p.v, p.sv, plane, p.H);
  const IO* __restrict__ G = plane_ptr<IO>(p.dout, p.sdo, plane, p.H);
  const float* __restrict__ tab = p.rope;
  const int shift = 1 - p.has_cls;
  const int64_t prow = (int64_t)plane * N;
  const float c2 = p.scale_log2;

  const int tid = thread_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int kv_first = kblk * KROWS + wave * 16;
  // transposed-read rows of staged query r (vperm: conflict-free in both directions)
  const int qt0 = vperm(8 * lg + (lr >> 2)), qt1 = vperm(8 * lg + 4 + (lr >> 2));

  // ---- tile start: the wave's K-hat / V rows, the tile's and plane's ranges ----
  float kx[KS][8], vy[KS][8];
  {
    const int row = kv_first + lr;
    const bool ok = row < N;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c = 32 * s + 8 * lg;
      if (ok) {
        float cs[8];
        load8(K + (int64_t)row * p.sk[2] + c, 1, true, kx[s]);
        rope_load4(tab, row + shift, D2, c / 2, cs);
        rope_rotate8(kx[s], cs);
        load8(V + (int64_t)row * p.sv[2] + c, 1, true, vy[s]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) kx[s][e] = vy[s][e] = 0.f;
      }
    }
  }
  {
    float amk = 0.f, vn2 = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      amk = amax8(amk, kx[s]);
#pragma unroll
      for (int e = 0; e < 8; ++e) vn2 = __builtin_fmaf(vy[s][e], vy[s][e], vn2);
    }
    const float vn = __builtin_sqrtf(group4_sum(vn2));   // |V_key|_2 of key lr
    // the plane's query rows: max |dO|_2, max |Q-hat * c2|, max |delta|
    float dmx = 0.f, qmx = 0.f, lmx = 0.f;
    for (int r = tid; r < N; r += NT) {
      const float2 st = reinterpret_cast<const float2*>(p.row_stat)[prow + r];
      dmx = fmaxf(dmx, st.x);
      qmx = fmaxf(qmx, st.y);
      lmx = fmaxf(lmx, fabsf(p.delta[prow + r]));
    }
    const unsigned w0 = wave_max_bits(amk), w1 = wave_max_bits(vn), w2 = wave_max_bits(dmx);
    const unsigned w3 = wave_max_bits(qmx), w4 = wave_max_bits(lmx);
    if (lane == 0) {
      sRed[wave][0] = __uint_as_float(w0);
      sRed[wave][1] = __uint_as_float(w1);
      sRed[wave][2] = __uint_as_float(w2);
      sRed[wave][3] = __uint_as_float(w3);
      sRed[wave][4] = __uint_as_float(w4);
    }
  }
  lds_barrier();
  float rk = 0.f, rv = 0.f, rd = 0.f, rq = 0.f, rl = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    rk = fmaxf(rk, sRed[w][0]);
    rv = fmaxf(rv, sRed[w][1]);
    rd = fmaxf(rd, sRed[w][2]);
    rq = fmaxf(rq, sRed[w][3]);
    rl = fmaxf(rl, sRed[w][4]);
  }
  const unsigned ek = __builtin_amdgcn_readfirstlane(__float_as_uint(rk)) >> 23;
  const unsigned eq = __builtin_amdgcn_readfirstlane(__float_as_uint(rq)) >> 23;
  // fp16 range of the logit operands (as the forward pass, plus a floor:
  // these rows are also the dK / dQ products' operands)
  const bool rescale = eq >= kF16ExpLimit || ek >= kF16ExpLimit || eq < kF16ExpLow || ek < kF16ExpLow;
  const float fq = rescale ? f16_fit(eq) : 1.f, fk = rescale ? f16_fit(ek) : 1.f;
  const float fsc = 1.f / (fq * fk);
  const bool raw = rescale;   // the prep kernel's fp16 rows are for fq = 1
  const float bound = __builtin_fmaf(rd, rv, rl);   // >= |dS| over the tile
  const float sig = f16_fit(__builtin_amdgcn_readfirstlane(__float_as_uint(bound)) >> 23);

  HFrag kf[KS];   // K-hat * fk: B operand of the logits (key lr, channels 32s + 8lg ..)
  Frag vf[KS];    // V * sig: B operand of dP
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    float x[8], y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = kx[s][e] * fk;
      y[e] = vy[s][e] * sig;
    }
    kf[s].v = to_f16x8(x);
    vf[s] = C::make(y);
  }
  // DS: this tile's K-hat * fk rows (rows >= N are zero) and its exponent of
  // 1 / (sig fk) for the dQ GEMM; sig dS^T is stored per query block below
  const int KP = p.n_blk * KROWS;
  if constexpr (DS) {
    f16* kh = static_cast<f16*>(p.khat) + ((int64_t)plane * KP + kv_first + lr) * D;
#pragma unroll
    for (int s = 0; s < KS; ++s) *reinterpret_cast<f16x8*>(kh + 32 * s + 8 * lg) = kf[s].v;
    if (tid == 0)
      p.kexp[plane * p.n_blk + kblk] = 254 - (int)(__float_as_uint(sig) >> 23) - (int)(__float_as_uint(fk) >> 23);
  }
  const auto rDS = make_rsrc(DS ? static_cast<const f16*>(p.ds_t) + (int64_t)plane * KP * p.nqp : nullptr,
                             DS ? (unsigned)(KP * p.nqp * 2) : 0u);

  f32x4 dvacc[DT], dkacc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) dvacc[d] = dkacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- stage staging (thread t, unit it: row c / CPR, channels 8 (c % CPR) ..) ----
  Raw8<f16> pqf[ITER];
  Raw8<IO> pg[ITER];
  float pl = 0.f, pd = 0.f;
  const auto rG = make_rsrc(G, (unsigned)(((int64_t)(N - 1) * p.sdo[2] + D) * ES));
  const auto rF = make_rsrc(static_cast<const f16*>(p.qhat_f) + prow * D, (unsigned)(N * D * 2));
  const auto rl_ = make_rsrc(p.lse + prow, (unsigned)N * 4u);
  const auto rd_ = make_rsrc(p.delta + prow, (unsigned)N * 4u);
  auto prefetch = [&](int qb) __attribute__((always_inline)) {
    if (!raw) {
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR;
        pqf[it] = buf_load8<f16>(rF, (unsigned)((r * D + 8 * cc) * 2), (unsigned)(qb * D * 2));
      }
    }
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int c = tid + it * NT;
      const int r = c / CPR, cc = c - r * CPR;
      pg[it] = buf_load8<IO>(rG, (unsigned)((r * (int)p.sdo[2] + 8 * cc) * (int)ES),
                             (unsigned)(qb * (int)p.sdo[2] * (int)ES));
    }
    if (tid < QS) {   // wave-uniform (QS is a multiple of 64)
      pl = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rl_, (unsigned)tid * 4u, (unsigned)qb * 4u, 0));
      pd = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rd_, (unsigned)tid * 4u, (unsigned)qb * 4u, 0));
    }
  };
  const float l2seed = kLog2e * fq * fk;
  auto commit = [&](int b, int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int c = tid + it * NT;
      const int r = c / CPR, cc = c - r * CPR;
      const int off = vperm(r) * LDQ + 8 * cc;
      if (!raw) {
        *reinterpret_cast<f16x8*>(&sQf[b][off]) = pqf[it].v;
      } else {
        // rescaled operands: rotate the row here (rows >= N are zero)
        const int gr = qb + r;
        float xq[8];
        if (gr < N) {
          float cs[8];
          load8(Q + (int64_t)gr * p.sq[2] + 8 * cc, 1, true, xq);
          rope_load4(tab, gr + shift, D2, 4 * cc, cs);
          rope_rotate8(xq, cs);
#pragma unroll
          for (int e = 0; e < 8; ++e) xq[e] *= c2 * fq;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) xq[e] = 0.f;
        }
        *reinterpret_cast<f16x8*>(&sQf[b][off]) = to_f16x8(xq);
      }
      if constexpr (std::is_same<IO, bf16>::value) {
        *reinterpret_cast<typename Raw8<IO>::vec*>(&sG[b][off]) = pg[it].v;
      } else {
        float xg[8];
        unpack8(pg[it], xg);
        C::put8(&sG[b][off], xg);
      }
    }
    if (tid < QS) {   // negated: they seed the S and dP accumulators
      sL2[b][tid] = qb + tid < N ? -pl * l2seed : -INFINITY;
      sDl[b][tid] = qb + tid < N ? -pd * sig : 0.f;
    }
  };

  // S and dP of query block j (32 queries) of the stage for the wave's keys;
  // query 32j + 8lg + 4h + i of accumulator h, element i (see the A rows).
  auto sp = [&](int b, int j, f32x4 (&sacc)[2], f32x4 (&pacc)[2]) __attribute__((always_inline)) {
    sacc[0] = *reinterpret_cast<const f32x4*>(&sL2[b][32 * j + 8 * lg]);
    sacc[1] = *reinterpret_cast<const f32x4*>(&sL2[b][32 * j + 8 * lg + 4]);
    pacc[0] = *reinterpret_cast<const f32x4*>(&sDl[b][32 * j + 8 * lg]);
    pacc[1] = *reinterpret_cast<const f32x4*>(&sDl[b][32 * j + 8 * lg + 4]);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int ql = 32 * j + vperm(8 * (lr >> 2) + 4 * h + (lr & 3));
        const HFrag a = H::lds(&sQf[b][ql * LDQ + 32 * s + 8 * lg]);
        const Frag g = C::lds(&sG[b][ql * LDQ + 32 * s + 8 * lg]);
        sacc[h] = H::mma(a, kf[s], sacc[h]);
        pacc[h] = C::mma(g, vf[s], pacc[h]);
      }
    }
  };
  // P and dS of block j, dV += P^T dO, dK-hat += (sig dS)^T Q-hat.  Keys >= N
  // have zero K-hat / V rows: their P is clamped to [0, 1], dS = -P delta is
  // finite and only reaches dK / dV rows that are never stored.
  auto pdk = [&](int b, int qb, int j, const f32x4 (&sacc)[2], const f32x4 (&pacc)[2]) __attribute__((always_inline)) {
    // the transposed operands of the first PF channel tiles are read before
    // the probabilities are formed, and each product then reads the tile PF
    // further on: every product waits for a read issued PF products earlier
    constexpr int PF = 3;
    Frag ag[DT];
    HFrag aq[DT];
    auto rd = [&](int d) __attribute__((always_inline)) {
      const int o0 = (32 * j + qt0) * LDQ + 16 * d + 4 * (lr & 3);
      const int o1 = (32 * j + qt1) * LDQ + 16 * d + 4 * (lr & 3);
      ag[d] = C::tr(&sG[b][o0], &sG[b][o1]);
      aq[d] = H::tr(&sQf[b][o0], &sQf[b][o1]);
    };
#pragma unroll
    for (int d = 0; d < PF; ++d) rd(d);
    float pv[8], dsv[8];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = __builtin_amdgcn_fmed3f(fast_exp2(sacc[h][i] * fsc), 0.f, 1.f);
        pv[4 * h + i] = pr;
        dsv[4 * h + i] = pr * pacc[h][i];
      }
    const Frag pf = C::make(pv);
    HFrag dsf;
    dsf.v = to_f16x8(dsv);
    if constexpr (DS) {   // sig dS^T: key kv_first + lr, queries qb + 32j + 8lg ..
      u32x4 w;
      __builtin_memcpy(&w, &dsf.v, 16);
      buf_store16(w, rDS, (unsigned)(((kv_first + lr) * p.nqp + qb + 32 * j + 8 * lg) * 2), 0u);
    }
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      // A = dO^T / Q-hat^T rows 16d.., k-slot e <-> query 32j + 8lg + e (the P / dS order)
      if (d + PF < DT) rd(d + PF);
      dvacc[d] = C::mma(ag[d], pf, dvacc[d]);
      dkacc[d] = H::mma(aq[d], dsf, dkacc[d]);
    }
  };
  prefetch(0);
  // One 64-query stage in buffer B (a compile-time constant: two stages per
  // trip, so the buffer addresses fold into the LDS instructions' offsets).
  auto stage = [&](int qb, auto bufc) __attribute__((always_inline)) {
    constexpr int B = decltype(bufc)::value;
    const int rows = min(QS, round_up32(N - qb));
    lds_barrier();   // this stage's commit (made during the previous stage) is visible
    // Two query blocks per trip: the S / dP products of block j+1 go to the
    // MFMA pipe before block j's probabilities are computed on the VALU (a
    // ragged last stage recomputes block j instead and skips its update).
    const int nbj = rows / 32;
    for (int j = 0; j < nbj; j += 2) {
      f32x4 sA[2], pA[2], sB[2], pB[2];
      sp(B, j, sA, pA);
      sp(B, min(j + 1, nbj - 1), sB, pB);
      pdk(B, qb, j, sA, pA);
      // the next stage goes into the other buffer (last read in the previous
      // stage, which every wave finished before this stage's barrier), and
      // the stage after it is prefetched (past the last stage: rows >= N)
      if (qb + QS < N) {
        commit(B ^ 1, qb + QS);
        prefetch(qb + 2 * QS);
      }
      if (j + 1 < nbj) {
        pdk(B, qb, j + 1, sB, pB);
        // the last block's order, which the scheduler otherwise collapses to
        // one read ahead: the 12 reads of its first three channel tiles, then
        // per tile its two products and the 4 reads three tiles on
        __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
          if (d + 3 < DT) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        }
        // (DS: the block's dS store after its products; first, it delays them)
        if constexpr (DS) __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
      }
    }
  };
  {
    commit(0, 0);
    prefetch(QS);
    int qb = 0;
    for (; qb + QS < N; qb += 2 * QS) {
      stage(qb, std::integral_constant<int, 0>{});
      stage(qb + QS, std::integral_constant<int, 1>{});
    }
    if (qb < N) stage(qb, std::integral_constant<int, 0>{});
  }

  // ---- epilogue: lane holds dV / dK-hat of key kv_first + lr, channels 16d + 4lg + (0..3) ----
  // 16 bytes per lane and store: lane groups lg and lg^1 trade halves
  // (v_permlane16_swap), so that even lg writes channels 16 d0 + 4 lg .. + 7
  // and odd lg channels 16 (d0 + 1) + 4 (lg - 1) .. + 7 for d0 = 0, 2, ...;
  // half the store instructions of 8-byte stores at the tile end, where the
  // workgroups of a launch round finish together.  Every lane takes part in
  // the exchange; rows >= N fall outside the descriptors' ranges.
  {
    const int row = kv_first + lr;
    const int trow = min(row, N - 1) + shift;   // (table row of a dropped row: any valid one)
    const auto rK = make_rsrc(plane_ptr<IO>(p.dk, p.sdk, plane, p.H), (unsigned)(((int64_t)(N - 1) * p.sdk[2] + D) * ES));
    const auto rV = make_rsrc(plane_ptr<IO>(p.dv, p.sdv, plane, p.H), (unsigned)(((int64_t)(N - 1) * p.sdv[2] + D) * ES));
    // dK-hat = scale * sum (sig dS)(Q-hat c2 fq) / (sig c2 fq)
    const float ks = p.scale / (sig * c2 * fq);
    typedef IO io4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int d0 = 0; d0 < DT; d0 += 2) {
      u32x2 wv[2], wk[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int d = d0 + h;
        float g4[4];
        io4 a, b;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          a[r] = (IO)dvacc[d][r];
          g4[r] = dkacc[d][r] * ks;
        }
        rope_unrotate4(g4, tab, trow, D2, 8 * d + 2 * lg);
#pragma unroll
        for (int r = 0; r < 4; ++r) b[r] = (IO)g4[r];
        __builtin_memcpy(&wv[h], &a, 8);
        __builtin_memcpy(&wk[h], &b, 8);
      }
      u32x4 xv, xk;
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const auto r1 = __builtin_amdgcn_permlane16_swap(wv[0][k], wv[1][k], false, false);
        xv[k] = r1[0];
        xv[2 + k] = r1[1];
        const auto r2 = __builtin_amdgcn_permlane16_swap(wk[0][k], wk[1][k], false, false);
        xk[k] = r2[0];
        xk[2 + k] = r2[1];
      }
      const int ch = 16 * (d0 + (lg & 1)) + 4 * (lg & 2);
      buf_store16(xv, rV, (unsigned)((row * (int)p.sdv[2] + ch) * (int)ES), 0u);
      buf_store16(xk, rK, (unsigned)((row * (int)p.sdk[2] + ch) * (int)ES), 0u);
    }
  }
}

hipError_t launch_bwd_keys(const BwdParams& p0, int io, hipStream_t st) {
  BwdParams p = p0;
  p.n_wg = p.B * p.H * p.n_blk;
  switch (io) {
    case DT_BF16:
      if (p.ds_t) hipLaunchKernelGGL((bwd_keys_kernel<bf16, true>), dim3(p.n_wg), dim3(512), 0, st, p);
      else hipLaunchKernelGGL((bwd_keys_kernel<bf16, false>), dim3(p.n_wg), dim3(512), 0, st, p);
      break;
    case DT_F16:
      if (p.ds_t) hipLaunchKernelGGL((bwd_keys_kernel<f16, true>), dim3(p.n_wg), dim3(512), 0, st, p);
      else hipLaunchKernelGGL((bwd_keys_kernel<f16, false>), dim3(p.n_wg), dim3(512), 0, st, p);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace farope
