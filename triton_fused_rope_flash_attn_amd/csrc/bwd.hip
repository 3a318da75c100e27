// Backward kernels for the fused 2D-RoPE attention.
//
// Reference behaviour followed ("fa_rope_full .py"):
//   delta = rowsum(dO * O) in fp32                      _attn_bwd_preprocess FA:325-357
//   P = exp(S - LSE), dV += P^T dO, dS = P*(dP - delta),
//   dK-hat += dS^T Q-hat, dK = R^T dK-hat * scale       _attn_bwd_dk_dv_rope FA:374-691
//   dQ-hat += dS K-hat,  dQ = R^T dQ-hat * scale        _attn_bwd_dq_rope    FA:708-1009
// with the CLS row bypassing the rotation (FA:647-662, FA:980-993).
//
// gfx950 design (fragment conventions in common.h):
//  * dK/dV kernel (KV-outer): each wave keeps its K-hat and V rows in
//    registers as B-operands.  Per 32-query block it computes S and dP
//    (query rows permuted so that lane group lg holds queries 8lg..8lg+7),
//    so P and dS land directly in the B-operand layout of
//    dV^T += dO^T P and dK-hat^T += Q-hat^T dS; dO^T and Q-hat^T are staged
//    transposed in LDS once per query stage and shared by all waves.
//  * For planes that fit on chip the one-pass kernel in bwd_fused.hip is
//    used instead; the kernels here serve any N and head_dim.
//  * dQ kernel (Q-outer, any N): logits transposed as in the forward pass;
//    dS^T lands in the B-operand layout of dQ-hat^T += K-hat^T dS^T.  It
//    can produce delta itself, so the split path needs no separate
//    preprocessing launch.
//  * Both kernels restage (load, rotate, write to LDS) the rows of the
//    other side of the plane for every workgroup, so workgroups are 8 waves
//    wide (BwdShape), and with vector-accessible inputs the next stage's raw
//    rows are prefetched into registers while the current one is computed.
//  * When 1 to 8 rows (keys) are left past the last full block, the launcher
//    runs these kernels over the full blocks only and tail.hip computes the
//    rest.
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O)  (fp32), one row per D/8 consecutive threads.
// ---------------------------------------------------------------------------
template <typename IO, int D>
__global__ void __launch_bounds__(256) bwd_pre_kernel(const BwdParams p) {
  constexpr int CPR = D / 8;
  constexpr int RPB = 256 / CPR;
  const int64_t grow = (int64_t)block_id() * RPB + thread_id() / CPR;
  const int cc = thread_id() % CPR;
  const int64_t total = (int64_t)p.B * p.H * p.N;
  float acc = 0.f;
  if (grow < total) {
    const int plane = (int)(grow / p.N);
    const int row = (int)(grow - (int64_t)plane * p.N);
    const int bb = plane / p.H, hh = plane - bb * p.H;
    const IO* O = static_cast<const IO*>(p.o) + bb * p.so[0] + hh * p.so[1] + row * p.so[2];
    const IO* G = static_cast<const IO*>(p.dout) + bb * p.sdo[0] + hh * p.sdo[1] + row * p.sdo[2];
    float o[8], g[8];
    load8(O + 8 * cc * p.so[3], p.so[3], p.vec_o, o);
    load8(G + 8 * cc * p.sdo[3], p.sdo[3], p.vec_do, g);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += o[e] * g[e];
    if (p.o_res) {   // O's rounding residual (contiguous [B, H, N, D])
      float r[8];
      load8(static_cast<const IO*>(p.o_res) + grow * D + 8 * cc, 1, true, r);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += r[e] * g[e];
    }
  }
#pragma unroll
  for (int m = 1; m < CPR; m <<= 1) acc += __shfl_xor(acc, m);
  if (grow < total && cc == 0) p.delta[grow] = acc;
}

// ---------------------------------------------------------------------------
// dQ kernel (Q-outer).
// ---------------------------------------------------------------------------
// VEC (K and V allow 16-byte access): the next KV block's raw rows are loaded
// into registers while the current block is computed (buffer descriptors over
// the plane, rows >= N read 0); their table rows are read when the block is
// committed.  Otherwise each block is loaded synchronously.
// FS (bf16 compute, head_dim >= 128): logits from fp16 operands as in the
// forward pass (the fp16 K-hat * fk tile in LDS, Q-hat in registers), and
// dQ-hat^T += (K-hat fk)^T (sig dS)^T with both operands in fp16 (one MFMA,
// 11 significant bits each).  A tile whose Q-hat or K-hat reaches 2^12 is
// computed again with scaled logit operands, and one whose largest |sig dS|
// left [2^-10, 2^15) (fp16 overflow, or values deep in its subnormal range)
// is computed again with sig = the power of two that puts it in
// [2^14, 2^15) (sig = 1 first).  Nothing is stored before a pass is kept.
// With p.row_stat the tile also writes each row's {|dO|_2, max |Q-hat c2|}
// for the key-tile kernel (bwd_keys.hip).
template <typename IO, int CT, int D, int NW, int QT, int KVS, bool WRITE_DELTA, bool VEC, bool FS>
__global__ void __launch_bounds__(NW * 64)
bwd_dq_kernel(const BwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  using LC = std::conditional_t<FS, Comp<DT_F16>, C>;   // logits operands
  using LFrag = typename LC::Frag;
  constexpr int KS = D / 32, DT = D / 16, D2 = D / 2;
  constexpr int PADE = 16 / sizeof(S);
  constexpr int LDK = D + PADE, LDT = KVS + PADE;
  constexpr int NT = NW * 64, CPR = D / 8;
  constexpr int ITER = (KVS * CPR + NT - 1) / NT;
  constexpr int QROWS = NW * QT * 16;
  // 16-bit operands: K-hat^T is read transposed from sK (ds_read_b64_tr_b16);
  // fp32 storage keeps an explicit transposed copy.
  constexpr bool TR = sizeof(S) == 2;

  static_assert(!FS || CT == DT_BF16, "fp16 logit operands go with bf16 compute");
  __shared__ __attribute__((aligned(16))) S sK[FS ? 8 : KVS * LDK];    // K-hat (non-FS)
  __shared__ __attribute__((aligned(16))) f16 sKf[FS ? KVS * LDK : 8];   // FS: fp16 K-hat * fk
  __shared__ __attribute__((aligned(16))) S sKt[TR ? 8 : D * LDT];
  __shared__ __attribute__((aligned(16))) S sV[KVS * LDK];
  __shared__ u32x4 sRange[FS ? NW : 1];   // FS: per-wave max |Q-hat|, |K-hat|, |sig dS| bits
  // XR: the plane's last row, when it is the only one past the full query
  // blocks (p.x_rows == 1), rides along one tile of the plane instead of a
  // tail kernel that would read the plane's K and V again.  Its logits, dP
  // and dQ run on the VALU against the staged key blocks: wave w takes keys
  // KVS/NW * w .. of each block and keeps a partial dQ row in LDS; the
  // partial rows are summed at the tile's end.  Its Q-hat (fp16, scaled
  // like the other rows and counted in the operand range), dO and delta are
  // staged once per pass.
  constexpr bool XR = FS && VEC && sizeof(IO) == 2 && KVS == 8 * NW;
  constexpr int XO = XR ? D / 64 : 1;   // dQ channels per lane (XR)
  __shared__ __attribute__((aligned(16))) f16 sXq[XR ? D : 8];
  __shared__ __attribute__((aligned(16))) S sXg[XR ? D : 8];
  __shared__ __attribute__((aligned(16))) float sXo[XR ? NW : 1][XR ? D : 4];
  __shared__ float sXd[2];   // delta, LSE2 of the last row
  // XR with p.xk_ws: per-wave sums of the last key's dK-hat and dV rows
  __shared__ __attribute__((aligned(16))) float sXk[XR ? NW : 1][XR ? 2 * D : 4];

  const int N = p.N;
  const int tile = xcd_remap(block_id(), p.n_wg);
  const int plane = tile / p.n_blk;
  const int qblk = tile - plane * p.n_blk;
  const bool xi = XR && p.x_rows != 0 && qblk == plane % p.n_blk;
  const int bb = plane / p.H, hh = plane - bb * p.H;
  const IO* __restrict__ Q = static_cast<const IO*>(p.q) + bb * p.sq[0] + hh * p.sq[1];
  const IO* __restrict__ K = static_cast<const IO*>(p.k) + bb * p.sk[0] + hh * p.sk[1];
  const IO* __restrict__ V = static_cast<const IO*>(p.v) + bb * p.sv[0] + hh * p.sv[1];
  const IO* __restrict__ O = static_cast<const IO*>(p.o) + bb * p.so[0] + hh * p.so[1];
  const IO* __restrict__ G = static_cast<const IO*>(p.dout) + bb * p.sdo[0] + hh * p.sdo[1];
  IO* __restrict__ dQ = static_cast<IO*>(p.dq) + bb * p.sdq[0] + hh * p.sdq[1];
  const float* __restrict__ tab = p.rope;
  const int shift = 1 - p.has_cls;
  const int64_t prow = (int64_t)plane * N;

  // FS: largest |Q-hat| (scaled) and |K-hat| this thread converted in the
  // current pass; the operand scales and the logit factor 1 / (fq fk) of a
  // rescaled pass (all 1 otherwise)
  float amax_q = 0.f, amax_k = 0.f, amax_s = 0.f;
  float fq = 1.f, fk = 1.f, fsc = 1.f, sig = 1.f;
  bool rescaled = false;
  int npass = 0;
  for (;;) {   // one pass, or up to three when FS rescales
  // (FS: the lane index is opaque to the compiler, so that no lane-dependent
  // address of the pass is hoisted out of this loop to hold registers)
  const int tid = FS ? opaque(thread_id()) : thread_id();
  const int wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  LFrag qf[QT][KS];
  Frag gf[QT][KS];
  float lse2[QT], dlt[QT];
  int qrow[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int row = qblk * QROWS + (wave * QT + t) * 16 + lr;
    qrow[t] = row;
    float dsum = 0.f, gn2 = 0.f, qmr = 0.f;   // (FS: the row statistics)
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c0 = 32 * s + 8 * lg;
      float x[8], g[8];
      if (row < N) {
        load8(Q + row * p.sq[2] + c0 * p.sq[3], p.sq[3], p.vec_q, x);
        float cs[8];
        rope_load4(tab, row + shift, D2, c0 / 2, cs);
        rope_rotate8(x, cs);
        load8(G + row * p.sdo[2] + c0 * p.sdo[3], p.sdo[3], p.vec_do, g);
        if (WRITE_DELTA) {
          float o[8];
          load8(O + row * p.so[2] + c0 * p.so[3], p.so[3], p.vec_o, o);
#pragma unroll
          for (int e = 0; e < 8; ++e) dsum += g[e] * o[e];
          if (p.o_res) {   // O's rounding residual (contiguous [B, H, N, D])
            load8(static_cast<const IO*>(p.o_res) + (prow + row) * D + c0, 1, true, o);
#pragma unroll
            for (int e = 0; e < 8; ++e) dsum += g[e] * o[e];
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = g[e] = 0.f;
      }
      if constexpr (FS) {
        // fp16 operands: Q-hat carries the logit scale (see put_khat)
        const float qs = p.scale_log2 * fq;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= qs;
        amax_q = amax8(amax_q, x);
        qf[t][s].v = to_f16x8(x);
        qmr = amax8(qmr, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) gn2 = __builtin_fmaf(g[e], g[e], gn2);
      } else {
        qf[t][s] = C::make(x);
      }
      gf[t][s] = C::make(g);
    }
    if constexpr (FS) {
      if (p.row_stat != nullptr && npass == 0) {   // (uniform; first pass: fq = 1)
        const float gn = __builtin_sqrtf(group4_sum(gn2)), qm = group4_max(qmr);
        if (lg == 0 && row < N) reinterpret_cast<float2*>(p.row_stat)[prow + row] = make_float2(gn, qm);
      }
    }
    if (WRITE_DELTA) {
      dsum = group4_sum(dsum);
      if (lg == 0 && row < N) p.delta[prow + row] = dsum;
      dlt[t] = dsum;
    } else {
      dlt[t] = row < N ? p.delta[prow + row] : 0.f;
    }
    lse2[t] = row < N ? p.lse[prow + row] * kLog2e : 0.f;
  }
  if constexpr (XR) {
    if (xi && wave == 0 && lane < D / 8) {
      const int row = N - 1, c0 = 8 * opaque(lane);
      float x[8], g[8], cs[8];
      load8(Q + row * p.sq[2] + c0 * p.sq[3], p.sq[3], p.vec_q, x);
      rope_load4(tab, row + shift, D2, c0 / 2, cs);
      rope_rotate8(x, cs);
      const float qs = p.scale_log2 * fq;
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= qs;
      amax_q = amax8(amax_q, x);
      *reinterpret_cast<f16x8*>(&sXq[c0]) = to_f16x8(x);
      if (p.qhat_f != nullptr && !rescaled)   // (see the tile rows' store below)
        *reinterpret_cast<f16x8*>(static_cast<f16*>(p.qhat_f) + (prow + row) * D + c0) = to_f16x8(x);
      load8(G + row * p.sdo[2] + c0 * p.sdo[3], p.sdo[3], p.vec_do, g);
      C::put8(&sXg[c0], g);
      if (p.row_stat != nullptr && npass == 0) {
        // over the D/8 active lanes, as delta below
        float gn2 = 0.f, qm = amax8(0.f, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) gn2 = __builtin_fmaf(g[e], g[e], gn2);
        gn2 = dpp_sum8(gn2);
        gn2 += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(gn2), 0x128, 0xF, 0xF, false));
        qm = fmaxf(qm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(qm), 0xB1, 0xF, 0xF, false)));
        qm = fmaxf(qm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(qm), 0x4E, 0xF, 0xF, false)));
        qm = fmaxf(qm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(qm), 0x141, 0xF, 0xF, false)));
        qm = fmaxf(qm, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(qm), 0x128, 0xF, 0xF, false)));
        if constexpr (D / 8 >= 32) {
          gn2 = xor16_pair_op_sum(gn2);
          qm = xor16_pair_op_max(qm);
        }
        if (lane == 0) reinterpret_cast<float2*>(p.row_stat)[prow + row] = make_float2(__builtin_sqrtf(gn2), qm);
      }
      float dsum;
      if (WRITE_DELTA) {
        float o[8];
        load8(O + row * p.so[2] + c0 * p.so[3], p.so[3], p.vec_o, o);
        dsum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) dsum += g[e] * o[e];
        if (p.o_res) {
          load8(static_cast<const IO*>(p.o_res) + (prow + row) * D + c0, 1, true, o);
#pragma unroll
          for (int e = 0; e < 8; ++e) dsum += g[e] * o[e];
        }
        // over the D/8 active lanes: 8-lane groups, then rows of 16, then row pairs
        dsum = dpp_sum8(dsum);
        dsum += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(dsum), 0x128, 0xF, 0xF, false));
        if constexpr (D / 8 >= 32) dsum = xor16_pair_op_sum(dsum);
        if (lane == 0) p.delta[prow + row] = dsum;
      } else {
        dsum = p.delta[prow + row];
      }
      if (lane == 0) {
        sXd[0] = dsum;
        sXd[1] = p.lse[prow + row] * kLog2e;
      }
    }
  }
  if constexpr (FS) amax_q = opaque(amax_q);
  const bool wave_active = qblk * QROWS + wave * QT * 16 < N;
  // K-hat is staged pre-scaled by scale * log2(e); with fp16 operands it is
  // staged times fk and the dQ product takes sig dS
  const float dq_scale = FS ? p.scale / (fk * sig) : p.scale / p.scale_log2;

  f32x4 dqacc[QT][DT];
#pragma unroll
  for (int t = 0; t < QT; ++t)
#pragma unroll
    for (int d = 0; d < DT; ++d) dqacc[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // K-hat row segment -> sK, pre-scaled by softmax_scale * log2(e) as in the
  // forward pass, so that both passes see bit-identical logits in log2 units
  // (dQ's scale divides it out again).  With fp16 operands every kernel
  // scales Q-hat instead, and K-hat goes to sKf in fp16 (times fk in a
  // rescaled pass), the operand of both the logits and the dQ products.
  auto put_khat = [&](int off, float (&xk)[8]) __attribute__((always_inline)) {
    if constexpr (!FS) {
#pragma unroll
      for (int e = 0; e < 8; ++e) xk[e] *= p.scale_log2;
      C::put8(&sK[off], xk);
    } else {
      if (rescaled) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xk[e] *= fk;
      }
      amax_k = opaque(amax8(amax_k, xk));   // (computed here, not at the tile's end)
      *reinterpret_cast<f16x8*>(&sKf[off]) = to_f16x8(xk);
    }
  };

  // ---- VEC: KV block prefetch registers (thread t: row t / CPR, channels
  //      8 (t % CPR) .. +7 of K and V) ----
  constexpr unsigned ES = sizeof(IO);
  static_assert(!VEC || (KVS * CPR) % NT == 0, "every thread stages whole units");
  Raw8<IO> pk[VEC ? ITER : 1], pv[VEC ? ITER : 1];
  // with one unit per thread the table rows are prefetched too
  constexpr bool TABPF = VEC && ITER == 1;
  f32x4 pt[2];
  auto prefetch = [&](int kvb) __attribute__((always_inline)) {
    if constexpr (VEC) {
      const auto rK = make_rsrc(K, (unsigned)(((int64_t)(N - 1) * p.sk[2] + D) * ES));
      const auto rV = make_rsrc(V, (unsigned)(((int64_t)(N - 1) * p.sv[2] + D) * ES));
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR;
        pk[it] = buf_load8<IO>(rK, (unsigned)((r * (int)p.sk[2] + 8 * cc) * (int)ES),
                               (unsigned)(kvb * (int)p.sk[2] * (int)ES));
        pv[it] = buf_load8<IO>(rV, (unsigned)((r * (int)p.sv[2] + 8 * cc) * (int)ES),
                               (unsigned)(kvb * (int)p.sv[2] * (int)ES));
        if constexpr (TABPF) {
          const f32x4* t = reinterpret_cast<const f32x4*>(tab + ((int64_t)(min(kvb + r, N - 1) + shift) * D2 + 4 * cc) * 2);
          pt[0] = t[0];
          pt[1] = t[1];
        }
      }
    }
  };
  auto commit = [&](int kvb) __attribute__((always_inline)) {
    if constexpr (VEC) {
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR;
        float xk[8], cs[8];
        unpack8(pk[it], xk);
        if constexpr (TABPF) {
#pragma unroll
          for (int e = 0; e < 4; ++e) { cs[e] = pt[0][e]; cs[4 + e] = pt[1][e]; }
        } else {
          rope_load4(tab, min(kvb + r, N - 1) + shift, D2, 4 * cc, cs);   // rows >= N are zero
        }
        rope_rotate8(xk, cs);
        put_khat(r * LDK + 8 * cc, xk);
        if constexpr (std::is_same<IO, S>::value) {
          *reinterpret_cast<typename Raw8<IO>::vec*>(&sV[r * LDK + 8 * cc]) = pv[it].v;
        } else {
          float xv[8];
          unpack8(pv[it], xv);
          C::put8(&sV[r * LDK + 8 * cc], xv);
        }
        if constexpr (!TR) {
#pragma unroll
          for (int e = 0; e < 8; ++e) C::put1(&sKt[(8 * cc + e) * LDT + r], xk[e]);
        }
      }
    }
  };

  prefetch(0);
  if constexpr (FS) {
    // First pass (fq = 1): the tile's fp16 Q-hat rows (scaled by c2) for the
    // dK/dV kernel, which then stages them instead of rotating Q again.
    // Issued after the first key block's loads, so that waiting for those
    // does not also wait for these stores.
    if (p.qhat_f != nullptr && !rescaled) {
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const int row = qrow[t];
        if (row < N) {
#pragma unroll
          for (int s = 0; s < KS; ++s)
            *reinterpret_cast<f16x8*>(static_cast<f16*>(p.qhat_f) + (prow + row) * D + 32 * s + 8 * lg) = qf[t][s].v;
        }
      }
    }
  }
  for (int kvb = 0; kvb < N; kvb += KVS) {
    const int rows = min(KVS, round_up32(N - kvb));
    if (kvb > 0) lds_barrier();
    if constexpr (VEC) {
      commit(kvb);
      lds_barrier();
      prefetch(kvb + KVS);   // past the last block: rows >= N, read as 0
      if (!wave_active) continue;
    } else {
    {
      float xk[ITER][8], xv[ITER][8], cs[ITER][8];
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR, gr = kvb + r;
        if (c < rows * CPR && gr < N) {
          load8(K + gr * p.sk[2] + 8 * cc * p.sk[3], p.sk[3], p.vec_k, xk[it]);
          load8(V + gr * p.sv[2] + 8 * cc * p.sv[3], p.sv[3], p.vec_v, xv[it]);
          rope_load4(tab, gr + shift, D2, 4 * cc, cs[it]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) { xk[it][e] = 0.f; xv[it][e] = 0.f; cs[it][e] = 0.f; }
        }
      }
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR;
        if (c < rows * CPR) {
          rope_rotate8(xk[it], cs[it]);
          put_khat(r * LDK + 8 * cc, xk[it]);
          C::put8(&sV[r * LDK + 8 * cc], xv[it]);
          if constexpr (!TR) {
#pragma unroll
            for (int e = 0; e < 8; ++e) C::put1(&sKt[(8 * cc + e) * LDT + r], xk[it][e]);
          }
        }
      }
    }
    lds_barrier();
    if (!wave_active) continue;
    }

    // Keys >= N (the rest of the block holding key N-1) need no mask: their
    // K-hat and V rows are zero, so S = dP = 0 there and P, dS are finite
    // (P is clamped to [0, 1], which the exact P never leaves, in the
    // exponential's own clamp bit), and their dS^T entries meet zero K-hat
    // rows in the dQ product.  The dP accumulators start at -delta of the
    // lane's query, so dP - delta needs no subtraction.
    // S (logits) and dP of key block j, as two separate product sets:
    auto s_of = [&](int j, f32x4 (&sacc)[QT][2]) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < QT; ++t) sacc[t][0] = sacc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kl = 32 * j + 8 * (lr >> 2) + 4 * h + (lr & 3);
          LFrag a;
          if constexpr (FS)
            a = LC::lds(&sKf[kl * LDK + 32 * s + 8 * lg]);
          else
            a = C::lds(&sK[kl * LDK + 32 * s + 8 * lg]);
#pragma unroll
          for (int t = 0; t < QT; ++t) sacc[t][h] = LC::mma(a, qf[t][s], sacc[t][h]);
        }
      }
    };
    auto p_of = [&](int j, f32x4 (&pacc)[QT][2]) __attribute__((always_inline)) {
#pragma unroll
      for (int t = 0; t < QT; ++t) pacc[t][0] = pacc[t][1] = f32x4{-dlt[t], -dlt[t], -dlt[t], -dlt[t]};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kl = 32 * j + 8 * (lr >> 2) + 4 * h + (lr & 3);
          const Frag b = C::lds(&sV[kl * LDK + 32 * s + 8 * lg]);
#pragma unroll
          for (int t = 0; t < QT; ++t) pacc[t][h] = C::mma(b, gf[t][s], pacc[t][h]);
        }
      }
    };
    // dS of key block j from its S / dP, then dQ-hat^T += K-hat^T dS^T:
    auto pq = [&](int j, const f32x4 (&sacc)[QT][2], const f32x4 (&pacc)[QT][2]) __attribute__((always_inline)) {
      using DFrag = std::conditional_t<FS, LFrag, Frag>;   // FS: sig dS in fp16
      DFrag dsf[QT];
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        float ds[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            ds[4 * h + i] = __builtin_amdgcn_fmed3f(
                                fast_exp2(FS ? __builtin_fmaf(sacc[t][h][i], fsc, -lse2[t])
                                             : sacc[t][h][i] - lse2[t]), 0.f, 1.f) * pacc[t][h][i];
        if constexpr (FS) {
#pragma unroll
          for (int e = 0; e < 8; ++e) ds[e] *= sig;
          amax_s = amax8(amax_s, ds);
          dsf[t].v = to_f16x8(ds);
        } else {
          dsf[t] = C::make(ds);
        }
      }
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        // A = K-hat^T rows 16d.., k-slot e <-> key 32j + 8lg + e (the dS^T order)
        if constexpr (FS) {
          const LFrag a = LC::tr(&sKf[tr_offset(32 * j + 8 * lg, 16 * d, LDK, lr)],
                                 &sKf[tr_offset(32 * j + 8 * lg + 4, 16 * d, LDK, lr)]);
#pragma unroll
          for (int t = 0; t < QT; ++t) dqacc[t][d] = LC::mma(a, dsf[t], dqacc[t][d]);
        } else {
          Frag a;
          if constexpr (TR)
            a = C::tr(&sK[tr_offset(32 * j + 8 * lg, 16 * d, LDK, lr)],
                      &sK[tr_offset(32 * j + 8 * lg + 4, 16 * d, LDK, lr)]);
          else
            a = C::lds(&sKt[(16 * d + lr) * LDT + 32 * j + 8 * lg]);
#pragma unroll
          for (int t = 0; t < QT; ++t) dqacc[t][d] = C::mma(a, dsf[t], dqacc[t][d]);
        }
      }
    };
    // Two key blocks per trip: the logits of block j+1 go to the MFMA pipe
    // before block j's dS is computed on the VALU, its dP after (two blocks'
    // S and dP accumulators together do not fit the registers).  A ragged
    // last block recomputes block j instead and skips its update.
    const int nbj = rows / 32;
    for (int j = 0; j < nbj; j += 2) {
      f32x4 sA[QT][2], pA[QT][2], sB[QT][2], pB[QT][2];
      s_of(j, sA);
      p_of(j, pA);
      s_of(min(j + 1, nbj - 1), sB);
      pq(j, sA, pA);
      p_of(min(j + 1, nbj - 1), pB);
      if (j + 1 < nbj) pq(j + 1, sB, pB);
    }
    if constexpr (XR) {
      if (xi) {
        // the last row against keys kvb + 8 * wave + (0..7): lane (key
        // lane / 8, channel slice lane % 8) forms the fp16 logit and the dP
        // dot products; every lane then adds the 8 dS-weighted K-hat rows
        // to channels XO * lane .. of the wave's partial dQ.  Keys >= N have
        // zero K-hat rows (no contribution), as in the block products.
        const int kk = lane >> 3, ds = lane & 7, r = 8 * wave + kk;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int i = 0; i < D / 64; ++i) {
          const int c = (D / 8) * ds + 8 * i;
          s = dot8<f16>(*reinterpret_cast<const Raw8<f16>*>(&sXq[c]), *reinterpret_cast<const Raw8<f16>*>(&sKf[r * LDK + c]), s);
          dp = dot8<S>(*reinterpret_cast<const Raw8<S>*>(&sXg[c]), *reinterpret_cast<const Raw8<S>*>(&sV[r * LDK + c]), dp);
        }
        s = dpp_sum8(s);
        dp = dpp_sum8(dp);
        const float dsx = __builtin_amdgcn_fmed3f(fast_exp2(__builtin_fmaf(s, fsc, -sXd[1])), 0.f, 1.f) * (dp - sXd[0]);
        float o[XO];
#pragma unroll
        for (int i = 0; i < XO; ++i) o[i] = kvb == 0 ? 0.f : sXo[wave][XO * lane + i];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float dj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(dsx), 8 * j));
          const f16* kb = &sKf[(8 * wave + j) * LDK + XO * lane];   // K-hat * fk
#pragma unroll
          for (int i = 0; i < XO; ++i) o[i] = __builtin_fmaf(dj, (float)kb[i], o[i]);
        }
#pragma unroll
        for (int i = 0; i < XO; ++i) sXo[wave][XO * lane + i] = o[i];
      }
    }
  }

  if constexpr (FS) {
    // Operand ranges of this pass over the workgroup; if Q-hat or K-hat
    // reached 2^12, run the tile again with scaled logit operands.
    {
      const unsigned rq = wave_max_bits(amax_q), rk = wave_max_bits(amax_k), rs = wave_max_bits(amax_s);
      if (lane == 0) sRange[wave] = u32x4{rq, rk, rs, 0u};
    }
    lds_barrier();
    unsigned rq = 0, rk = 0, rs = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const u32x4 r = sRange[w];
      rq = max(rq, r[0]);
      rk = max(rk, r[1]);
      rs = max(rs, r[2]);
    }
    const unsigned eq = __builtin_amdgcn_readfirstlane(rq) >> 23;
    const unsigned ek = __builtin_amdgcn_readfirstlane(rk) >> 23;
    const unsigned es = __builtin_amdgcn_readfirstlane(rs) >> 23;
    // logit operands past 2^12 (once), or sig dS outside [2^-10, 2^15)
    // (es == 0: every dS is zero); at most three passes
    const bool redo_l = !rescaled && (eq >= kF16ExpLimit || ek >= kF16ExpLimit);
    const bool redo_s = es >= 142u || (es != 0u && es < 117u);
    if ((redo_l || redo_s) && npass < 2) {
      ++npass;
      if (redo_l) {
        rescaled = true;
        fq = f16_fit(eq);
        fk = f16_fit(ek);
        fsc = 1.f / (fq * fk);
      }
      // (a max of inf / NaN keeps sig: f16_fit(255) would flush every value)
      if (redo_s && es < 255u) sig *= f16_fit(es);
      amax_q = amax_k = amax_s = 0.f;
      continue;
    }
  }
  if constexpr (XR) {
    // (the range barrier above ordered every wave's partial dQ row)
    if (xi && wave == 0 && lane < D / 4) {
      const int ln = opaque(lane);   // (addresses formed here, not kept through the pass)
      float g4[4] = {};
#pragma unroll
      for (int w = 0; w < NW; ++w)
#pragma unroll
        for (int r = 0; r < 4; ++r) g4[r] += sXo[w][4 * ln + r];
#pragma unroll
      for (int r = 0; r < 4; ++r) g4[r] *= p.scale / fk;   // (K-hat * fk, fp32 dS)
      rope_unrotate4(g4, tab, N - 1 + shift, D2, 2 * ln);
      store4(dQ + (N - 1) * p.sdq[2] + 4 * ln * p.sdq[3], p.sdq[3], p.vec_dq, g4);
    }
  }

#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int row = FS ? opaque(qrow[t]) : qrow[t];   // (FS: table address formed here)
    if (row < N) {
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        float g4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) g4[r] = dqacc[t][d][r] * dq_scale;
        rope_unrotate4(g4, tab, row + shift, D2, 8 * d + 2 * lg);
        store4(dQ + row * p.sdq[2] + (16 * d + 4 * lg) * p.sdq[3], p.sdq[3], p.vec_dq, g4);
      }
    }
  }
  if constexpr (XR) {
    if (p.xk_ws) {
      // The plane's last key (the one key past the dK/dV kernel's full key
      // blocks): its dK-hat and dV rows summed over this tile's query rows,
      // from the tile's Q-hat / dO fragments and the key's K-hat / V row,
      // which the last key block left in LDS (row er).  P and dS as in the
      // block products (exp2(S - LSE2) clamped to [0, 1]; rows >= N have
      // zero fragments and add nothing).  Each tile writes one partial row
      // pair; bwd_tail_key_merge_kernel adds the tiles' rows in a fixed
      // order.  dK-hat is summed against the fp16 Q-hat (scaled by c2 * fq)
      // and divided by that scale here.
      const int er = (N - 1) % KVS;
      const int ln = opaque(lane);
      const int lgx = ln >> 4, lrx = ln & 15;
      float prx[QT], dsx[QT];
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        float sx = 0.f, dpx = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int c0 = 32 * s + 8 * lgx;
          Raw8<f16> a;
          a.v = opaque_vec(qf[t][s].v);
          Raw8<S> b;
          b.v = opaque_vec(gf[t][s].v);
          sx = dot8<f16>(a, *reinterpret_cast<const Raw8<f16>*>(&sKf[er * LDK + c0]), sx);
          dpx = dot8<S>(b, *reinterpret_cast<const Raw8<S>*>(&sV[er * LDK + c0]), dpx);
        }
        sx = group4_sum(sx);
        dpx = group4_sum(dpx);
        prx[t] = __builtin_amdgcn_fmed3f(fast_exp2(__builtin_fmaf(sx, fsc, -lse2[t])), 0.f, 1.f);
        dsx[t] = prx[t] * (dpx - dlt[t]);
      }
      // each channel's products over the lane's query rows, then the sum over
      // the 16 query rows of each lane group (DPP within rows of 16)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        decltype(qf[0][0].v) qv[QT];
        decltype(gf[0][0].v) gv[QT];
#pragma unroll
        for (int t = 0; t < QT; ++t) {
          qv[t] = opaque_vec(qf[t][s].v);
          gv[t] = opaque_vec(gf[t][s].v);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x = 0.f, y = 0.f;
#pragma unroll
          for (int t = 0; t < QT; ++t) {
            x = __builtin_fmaf(dsx[t], (float)qv[t][e], x);
            y = __builtin_fmaf(prx[t], (float)gv[t][e], y);
          }
          x = dpp_sum8(x);
          y = dpp_sum8(y);
          x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
          y += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(y), 0x140, 0xF, 0xF, false));
          if (lrx == 0) {
            sXk[wave][32 * s + 8 * lgx + e] = x;
            sXk[wave][D + 32 * s + 8 * lgx + e] = y;
          }
        }
      }
      lds_barrier();
      if (wave == 0) {
        // the tile's last row (XR item): its own products with the key
        float px = 0.f, dsxx = 0.f;
        if (xi) {
          float s1 = 0.f, d1 = 0.f;
#pragma unroll
          for (int i = 0; i < XO; ++i) {
            const int c = XO * ln + i;
            s1 = __builtin_fmaf((float)sXq[c], (float)sKf[er * LDK + c], s1);
            d1 = __builtin_fmaf((float)sXg[c], (float)sV[er * LDK + c], d1);
          }
          s1 = dpp_sum8(s1);
          d1 = dpp_sum8(d1);
          s1 += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s1), 0x140, 0xF, 0xF, false));
          d1 += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(d1), 0x140, 0xF, 0xF, false));
          s1 = group4_sum(s1);
          d1 = group4_sum(d1);
          px = __builtin_amdgcn_fmed3f(fast_exp2(__builtin_fmaf(s1, fsc, -sXd[1])), 0.f, 1.f);
          dsxx = px * (d1 - sXd[0]);
        }
        const float iq = 1.f / (p.scale_log2 * fq);
        float* ws = p.xk_ws + ((int64_t)plane * p.n_blk + qblk) * (2 * D);
#pragma unroll
        for (int m = 0; m < 2 * D / 64; ++m) {
          const int j = ln + 64 * m;
          float x = 0.f;
#pragma unroll
          for (int w = 0; w < NW; ++w) x += sXk[w][j];
          if (j < D) {
            if (xi) x = __builtin_fmaf(dsxx, (float)sXq[j], x);
            x *= iq;
          } else {
            if (xi) x = __builtin_fmaf(px, (float)sXg[j - D], x);
          }
          ws[j] = x;
        }
      }
    }
  }
  break;
  }   // pass
}

// ---------------------------------------------------------------------------
// dK/dV kernel (KV-outer).
// ---------------------------------------------------------------------------
// VEC (Q and dO allow 16-byte access, decided on the host): the rows of the
// next query stage are loaded into registers while the current stage is
// computed, through buffer descriptors over the plane (rows >= N read 0), and
// committed to LDS after the stage barrier.  Otherwise each stage is loaded
// element-wise and synchronously.
// FS (bf16 compute, head_dim >= 128): logits from fp16 operands (an fp16
// Q-hat tile next to the bf16 one the dK product reads; K-hat in registers),
// and dK-hat^T += Q-hat^T dS_hi + Q-hat^T dS_lo.  A tile whose Q-hat or K-hat
// reaches 2^12 is computed again with scaled logit operands.
// HAT (FS, VEC): the stage's Q-hat rows come rotated from the dQ kernel's
// first pass (p.qhat_f: fp16 of Q-hat * c2), so a stage loads one 16-byte
// row segment per unit instead of the Q row and its 32 bytes of table; the
// bf16 Q-hat of the dK product is that value divided by c2.  A pass whose
// fp16 rows overflowed (inf) or underflowed (max below 2^-10) rotates Q
// again (raw), and a rescaled pass does too.
template <typename IO, int CT, int D, int NW, int KT, int QS, bool VEC, bool FS, bool HAT>
__global__ void __launch_bounds__(NW * 64)
bwd_dkdv_kernel(const BwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  using LC = std::conditional_t<FS, Comp<DT_F16>, C>;   // logits operands
  using LFrag = typename LC::Frag;
  constexpr int KS = D / 32, DT = D / 16, D2 = D / 2;
  constexpr int PADE = 16 / sizeof(S);
  constexpr int LDQ = D + PADE, LDT = QS + PADE;
  constexpr int NT = NW * 64, CPR = D / 8;
  constexpr int ITER = (QS * CPR + NT - 1) / NT;
  constexpr int KROWS = NW * KT * 16;           // kv rows per workgroup
  // 16-bit operands: Q-hat^T and dO^T are read transposed from sQ / sG
  // (ds_read_b64_tr_b16); fp32 storage keeps explicit transposed copies.
  constexpr bool TR = sizeof(S) == 2;

  static_assert(!FS || CT == DT_BF16, "fp16 logit operands go with bf16 compute");
  __shared__ __attribute__((aligned(16))) S sQ[QS * LDQ];
  __shared__ __attribute__((aligned(16))) f16 sQf[FS ? QS * LDQ : 8];   // FS: fp16 Q-hat (scaled)
  __shared__ u32x2 sRange[FS ? NW : 1];   // FS: per-wave max |Q-hat|, |K-hat| bits
  __shared__ __attribute__((aligned(16))) S sQt[TR ? 8 : D * LDT];
  __shared__ __attribute__((aligned(16))) S sG[QS * LDQ];
  __shared__ __attribute__((aligned(16))) S sGt[TR ? 8 : D * LDT];
  __shared__ __attribute__((aligned(16))) float sL2[QS];
  __shared__ __attribute__((aligned(16))) float sDl[QS];

  const int N = p.N;
  const int tile = xcd_remap(block_id(), p.n_wg);
  const int plane = tile / p.n_blk;
  const int kblk = tile - plane * p.n_blk;
  const int bb = plane / p.H, hh = plane - bb * p.H;
  const IO* __restrict__ Q = static_cast<const IO*>(p.q) + bb * p.sq[0] + hh * p.sq[1];
  const IO* __restrict__ K = static_cast<const IO*>(p.k) + bb * p.sk[0] + hh * p.sk[1];
  const IO* __restrict__ V = static_cast<const IO*>(p.v) + bb * p.sv[0] + hh * p.sv[1];
  const IO* __restrict__ G = static_cast<const IO*>(p.dout) + bb * p.sdo[0] + hh * p.sdo[1];
  IO* __restrict__ dK = static_cast<IO*>(p.dk) + bb * p.sdk[0] + hh * p.sdk[1];
  IO* __restrict__ dV = static_cast<IO*>(p.dv) + bb * p.sdv[0] + hh * p.sdv[1];
  const float* __restrict__ tab = p.rope;
  const int shift = 1 - p.has_cls;
  const int64_t prow = (int64_t)plane * N;

  // FS: largest |Q-hat| (scaled) and |K-hat| this thread converted in the
  // current pass; the operand scales and the logit factor 1 / (fq fk) of a
  // rescaled pass (all 1 otherwise)
  float amax_q = 0.f, amax_k = 0.f;
  float fq = 1.f, fk = 1.f, fsc = 1.f;
  bool rescaled = false;
  // HAT: a pass that rotates Q itself because the dQ kernel's fp16 rows hid
  // the operand range
  bool raw = false;
  const float ic2 = 1.f / p.scale_log2;
  for (;;) {   // one pass, or two when FS rescales
  // (FS: the lane index is opaque to the compiler, so that no lane-dependent
  // address of the pass is hoisted out of this loop to hold registers)
  const int tid = FS ? opaque(thread_id()) : thread_id();
  const int wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int kv_first = kblk * KROWS + wave * KT * 16;
  // 16-bit tiles: LDS row of staged query r (see vperm: conflict-free
  // transposed reads), and the rows of the lane's two transposed reads
  auto qrow = [](int r) { return TR ? vperm(r) : r; };
  const int qt0 = qrow(8 * lg + (lr >> 2)), qt1 = qrow(8 * lg + 4 + (lr >> 2));
  // LSE (natural log) -> the S accumulators' seed -LSE2 (FS: times fq fk)
  const float l2seed = FS ? kLog2e * fq * fk : kLog2e;
  // ---- this wave's K-hat and V rows as B-operands ----
  LFrag kf[KT][KS];
  Frag vf[KT][KS];
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    const int row = kv_first + 16 * u + lr;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c0 = 32 * s + 8 * lg;
      float x[8], y[8];
      if (row < N) {
        load8(K + row * p.sk[2] + c0 * p.sk[3], p.sk[3], p.vec_k, x);
        float cs[8];
        rope_load4(tab, row + shift, D2, c0 / 2, cs);
        rope_rotate8(x, cs);
        // pre-scaled by softmax_scale * log2(e), as every kernel stages K-hat
        // (fp16 operands: Q-hat carries the scale; K-hat times fk)
        const float ks = FS ? fk : p.scale_log2;
        if (!FS || rescaled) {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] *= ks;
        }
        load8(V + row * p.sv[2] + c0 * p.sv[3], p.sv[3], p.vec_v, y);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = y[e] = 0.f;
      }
      if constexpr (FS) {
        amax_k = amax8(amax_k, x);
        kf[u][s].v = to_f16x8(x);
      } else {
        kf[u][s] = C::make(x);
      }
      vf[u][s] = C::make(y);
    }
  }
  if constexpr (FS) amax_k = opaque(amax_k);

  f32x4 dvacc[KT][DT], dkacc[KT][DT];
#pragma unroll
  for (int u = 0; u < KT; ++u)
#pragma unroll
    for (int d = 0; d < DT; ++d) dvacc[u][d] = dkacc[u][d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Q-hat row segment -> sQ (FS: also Q-hat * scale * log2(e) * fq to sQf in fp16)
  auto put_qhat = [&](int off, const float (&xq)[8]) __attribute__((always_inline)) {
    C::put8(&sQ[off], xq);
    if constexpr (FS) {
      const float qs = p.scale_log2 * fq;
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = xq[e] * qs;
      amax_q = opaque(amax8(amax_q, x));   // (computed here, not at the tile's end)
      *reinterpret_cast<f16x8*>(&sQf[off]) = to_f16x8(x);
    }
  };

  // ---- VEC: stage prefetch registers (thread t: row t / CPR, channels
  //      8 (t % CPR) .. +7 of Q and dO, their table row; threads t < QS: LSE
  //      and delta of row t) ----
  constexpr unsigned ES = sizeof(IO);
  static_assert(!VEC || (QS * CPR) % NT == 0, "every thread stages whole units");
  static_assert(!VEC || QS <= NT, "one thread per staged LSE / delta");
  static_assert(!HAT || (FS && VEC), "rotated rows come with fp16 logits and vector access");
  Raw8<IO> pq[VEC && !HAT ? ITER : 1], pg[VEC ? ITER : 1];
  f32x4 pt[VEC && !HAT ? ITER : 1][2];
  Raw8<f16> pqf[HAT ? ITER : 1];
  float pl = 0.f, pd = 0.f;
  auto prefetch = [&](int qb) __attribute__((always_inline)) {
    if constexpr (VEC) {
      const auto rG = make_rsrc(G, (unsigned)(((int64_t)(N - 1) * p.sdo[2] + D) * ES));
      if constexpr (HAT) {
        if (!rescaled && !raw) {   // (otherwise commit rotates Q itself)
          const auto rF = make_rsrc(static_cast<const f16*>(p.qhat_f) + prow * D, (unsigned)(N * D * 2));
#pragma unroll
          for (int it = 0; it < ITER; ++it) {
            const int c = tid + it * NT;
            const int r = c / CPR, cc = c - r * CPR;
            pqf[it] = buf_load8<f16>(rF, (unsigned)((r * D + 8 * cc) * 2), (unsigned)(qb * D * 2));
          }
        }
      } else {
        const auto rQ = make_rsrc(Q, (unsigned)(((int64_t)(N - 1) * p.sq[2] + D) * ES));
#pragma unroll
        for (int it = 0; it < ITER; ++it) {
          const int c = tid + it * NT;
          const int r = c / CPR, cc = c - r * CPR;
          pq[it] = buf_load8<IO>(rQ, (unsigned)((r * (int)p.sq[2] + 8 * cc) * (int)ES),
                                 (unsigned)(qb * (int)p.sq[2] * (int)ES));
          // rows >= N are zero; any table row serves them
          const f32x4* t = reinterpret_cast<const f32x4*>(tab + ((int64_t)(min(qb + r, N - 1) + shift) * D2 + 4 * cc) * 2);
          pt[it][0] = t[0];
          pt[it][1] = t[1];
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
        const auto rl = make_rsrc(p.lse + prow, (unsigned)N * 4u);
        const auto rd = make_rsrc(p.delta + prow, (unsigned)N * 4u);
        pl = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rl, (unsigned)tid * 4u, (unsigned)qb * 4u, 0));
        pd = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rd, (unsigned)tid * 4u, (unsigned)qb * 4u, 0));
      }
    }
  };
  auto commit = [&](int qb) __attribute__((always_inline)) {
    if constexpr (VEC) {
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR;
        float xq[8], xg[8];
        unpack8(pg[it], xg);
        if constexpr (HAT) {
          if (!rescaled && !raw) {
            // the dQ pass's rotated rows (rows >= N read 0)
            *reinterpret_cast<f16x8*>(&sQf[qrow(r) * LDQ + 8 * cc]) = pqf[it].v;
            float xf[8];
            unpack8(pqf[it], xf);
            amax_q = opaque(amax8(amax_q, xf));
#pragma unroll
            for (int e = 0; e < 8; ++e) xf[e] *= ic2;
            C::put8(&sQ[qrow(r) * LDQ + 8 * cc], xf);
          } else {
            const int gr = qb + r;
            if (gr < N) {
              float cs[8];
              load8(Q + gr * p.sq[2] + 8 * cc * p.sq[3], p.sq[3], true, xq);
              rope_load4(tab, gr + shift, D2, 4 * cc, cs);
              rope_rotate8(xq, cs);
            } else {
#pragma unroll
              for (int e = 0; e < 8; ++e) xq[e] = 0.f;
            }
            put_qhat(qrow(r) * LDQ + 8 * cc, xq);
          }
        } else {
          unpack8(pq[it], xq);
          const float cs[8] = {pt[it][0][0], pt[it][0][1], pt[it][0][2], pt[it][0][3],
                               pt[it][1][0], pt[it][1][1], pt[it][1][2], pt[it][1][3]};
          rope_rotate8(xq, cs);
          put_qhat(qrow(r) * LDQ + 8 * cc, xq);
        }
        C::put8(&sG[qrow(r) * LDQ + 8 * cc], xg);
        if constexpr (!TR) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            C::put1(&sQt[(8 * cc + e) * LDT + r], xq[e]);
            C::put1(&sGt[(8 * cc + e) * LDT + r], xg[e]);
          }
        }
      }
      if (tid < QS) {   // negated: they seed the S and dP accumulators
        sL2[tid] = qb + tid < N ? -pl * l2seed : -INFINITY;
        sDl[tid] = qb + tid < N ? -pd : 0.f;
      }
    }
  };

  prefetch(0);
  for (int qb = 0; qb < N; qb += QS) {
    const int rows = min(QS, round_up32(N - qb));
    lds_barrier();
    if constexpr (VEC) {
      commit(qb);
      lds_barrier();
      prefetch(qb + QS);   // past the last stage: rows >= N, read as 0
    } else {
    // ---- stage Q-hat, Q-hat^T, dO, dO^T (+ delta, LSE) for this q stage ----
    {
      float xq[ITER][8], xg[ITER][8], cs[ITER][8];
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR, gr = qb + r;
        if (c < rows * CPR && gr < N) {
          load8(Q + gr * p.sq[2] + 8 * cc * p.sq[3], p.sq[3], p.vec_q, xq[it]);
          load8(G + gr * p.sdo[2] + 8 * cc * p.sdo[3], p.sdo[3], p.vec_do, xg[it]);
          rope_load4(tab, gr + shift, D2, 4 * cc, cs[it]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) { xq[it][e] = xg[it][e] = cs[it][e] = 0.f; }
        }
      }
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int c = tid + it * NT;
        const int r = c / CPR, cc = c - r * CPR;
        if (c < rows * CPR) {
          rope_rotate8(xq[it], cs[it]);
          put_qhat(qrow(r) * LDQ + 8 * cc, xq[it]);
          C::put8(&sG[qrow(r) * LDQ + 8 * cc], xg[it]);
          if constexpr (!TR) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              C::put1(&sQt[(8 * cc + e) * LDT + r], xq[it][e]);
              C::put1(&sGt[(8 * cc + e) * LDT + r], xg[it][e]);
            }
          }
        }
      }
      for (int r = tid; r < rows; r += NT) {
        const int gr = qb + r;
        sL2[r] = gr < N ? -p.lse[prow + gr] * l2seed : -INFINITY;
        sDl[r] = gr < N ? -p.delta[prow + gr] : 0.f;
      }
    }
    lds_barrier();
    }

    // S and dP of query block j for key subtile u.  -LSE2 and -delta of
    // queries 32j + 8lg + e, e = 4h + i, seed the accumulators of half h
    // (P = exp2(S), dP - delta need no arithmetic; queries >= N have
    // -LSE2 = -inf, so P = 0).
    auto sp = [&](int j, int u, f32x4 (&sacc)[2], f32x4 (&pacc)[2]) __attribute__((always_inline)) {
        sacc[0] = *reinterpret_cast<const f32x4*>(&sL2[32 * j + 8 * lg]);
        sacc[1] = *reinterpret_cast<const f32x4*>(&sL2[32 * j + 8 * lg + 4]);
        pacc[0] = *reinterpret_cast<const f32x4*>(&sDl[32 * j + 8 * lg]);
        pacc[1] = *reinterpret_cast<const f32x4*>(&sDl[32 * j + 8 * lg + 4]);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int ql = 32 * j + qrow(8 * (lr >> 2) + 4 * h + (lr & 3));
            LFrag a;
            if constexpr (FS)
              a = LC::lds(&sQf[ql * LDQ + 32 * s + 8 * lg]);
            else
              a = C::lds(&sQ[ql * LDQ + 32 * s + 8 * lg]);
            const Frag b = C::lds(&sG[ql * LDQ + 32 * s + 8 * lg]);
            sacc[h] = LC::mma(a, kf[u][s], sacc[h]);
            pacc[h] = C::mma(b, vf[u][s], pacc[h]);
          }
        }
    };
    // P and dS of query block j from its S / dP, then dV += P dO and
    // dK-hat += dS Q-hat for key subtile u.
    auto pdk = [&](int j, int u, const f32x4 (&sacc)[2], const f32x4 (&pacc)[2]) __attribute__((always_inline)) {
        // Keys >= N (lane key kv0 + lr) need no mask: their K-hat and V rows
        // are zero, so P and dS there are finite and only reach the dK / dV
        // rows of those keys, which are never stored.
        float pv[8], dsv[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int e = 4 * h + i;
            // FS: the seeds are -LSE2 * fq * fk, so this is exp2(S - LSE2)
            const float pr = fast_exp2(FS ? sacc[h][i] * fsc : sacc[h][i]);
            pv[e] = pr;
            dsv[e] = pr * pacc[h][i];
          }
        const Frag pf = C::make(pv);
        Frag dsf, dsfl;
        if constexpr (FS)
          split_bf16x8(dsv, dsf.v, dsfl.v);
        else
          dsf = C::make(dsv);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          // A = dO^T / Q-hat^T rows 16d.., k-slot e <-> query 32j + 8lg + e (the P / dS order)
          Frag ag, aq;
          if constexpr (TR) {
            const int o0 = (32 * j + qt0) * LDQ + 16 * d + 4 * (lr & 3);
            const int o1 = (32 * j + qt1) * LDQ + 16 * d + 4 * (lr & 3);
            ag = C::tr(&sG[o0], &sG[o1]);
            aq = C::tr(&sQ[o0], &sQ[o1]);
          } else {
            ag = C::lds(&sGt[(16 * d + lr) * LDT + 32 * j + 8 * lg]);
            aq = C::lds(&sQt[(16 * d + lr) * LDT + 32 * j + 8 * lg]);
          }
          dvacc[u][d] = C::mma(ag, pf, dvacc[u][d]);
          if constexpr (FS) dkacc[u][d] = C::mma(aq, dsfl, dkacc[u][d]);
          dkacc[u][d] = C::mma(aq, dsf, dkacc[u][d]);
        }
    };

    if constexpr (KT == 1 && sizeof(S) == 2) {
      // Two query blocks per trip: the S / dP products of block j+1 go to the
      // MFMA pipe before block j's probabilities are computed on the VALU (a
      // ragged last block recomputes block j instead and skips its update).
      if (kv_first < N) {   // wave-uniform
        const int nbj = rows / 32;
        for (int j = 0; j < nbj; j += 2) {
          f32x4 sA[2], pA[2], sB[2], pB[2];
          sp(j, 0, sA, pA);
          sp(min(j + 1, nbj - 1), 0, sB, pB);
          pdk(j, 0, sA, pA);
          if (j + 1 < nbj) pdk(j + 1, 0, sB, pB);
        }
      }
    } else {
      for (int j = 0; j < rows / 32; ++j) {
#pragma unroll
        for (int u = 0; u < KT; ++u) {
          if (kv_first + 16 * u >= N) continue;   // wave-uniform
          f32x4 sacc[2], pacc[2];
          sp(j, u, sacc, pacc);
          pdk(j, u, sacc, pacc);
        }
      }
    }
  }

  if constexpr (FS) {
    // Operand ranges of this pass over the workgroup; if Q-hat or K-hat
    // reached 2^12, run the tile again with scaled logit operands.
    {
      const unsigned rq = wave_max_bits(amax_q), rk = wave_max_bits(amax_k);
      if (lane == 0) sRange[wave] = u32x2{rq, rk};
    }
    lds_barrier();
    unsigned rq = 0, rk = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const u32x2 r = sRange[w];
      rq = max(rq, r[0]);
      rk = max(rk, r[1]);
    }
    const unsigned eq = __builtin_amdgcn_readfirstlane(rq) >> 23;
    const unsigned ek = __builtin_amdgcn_readfirstlane(rk) >> 23;
    if constexpr (HAT) {
      // fp16 rows of the dQ pass that overflowed (inf) or are all below
      // 2^-10 (their bf16 Q-hat would lose precision): the same pass from Q
      if (!raw && !rescaled && (eq >= 255u || eq < 117u)) {
        raw = true;
        amax_q = amax_k = 0.f;
        continue;
      }
    }
    if (!rescaled && (eq >= kF16ExpLimit || ek >= kF16ExpLimit)) {
      rescaled = true;
      fq = f16_fit(eq);
      fk = f16_fit(ek);
      fsc = 1.f / (fq * fk);
      amax_q = amax_k = 0.f;
      continue;
    }
  }

  // ---- epilogue: lane holds dV / dK-hat of kv row kv0 + lr, channels 16d + 4lg + (0..3) ----
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    const int row = kv_first + 16 * u + lr;
    if (row < N) {
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        float v4[4], g4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) { v4[r] = dvacc[u][d][r]; g4[r] = dkacc[u][d][r] * p.scale; }
        store4(dV + row * p.sdv[2] + (16 * d + 4 * lg) * p.sdv[3], p.sdv[3], p.vec_dv, v4);
        rope_unrotate4(g4, tab, row + shift, D2, 8 * d + 2 * lg);
        store4(dK + row * p.sdk[2] + (16 * d + 4 * lg) * p.sdk[3], p.sdk[3], p.vec_dk, g4);
      }
    }
  }
  break;
  }   // pass
}

// ---------------------------------------------------------------------------
// Tile table for the backward pass.
// ---------------------------------------------------------------------------
// Rows per workgroup: the Q / dO (dK/dV kernel) and K / V (dQ kernel) rows
// staged per workgroup are rotated and written to LDS once for all of its
// waves, so wider workgroups amortise that staging over more keys / queries
// (8 waves instead of 4: -29% at N = 1025, D = 128; two query subtiles per
// dQ wave: another -13%).  fp32 compute splits every operand into two bf16
// halves and needs the smaller tiles to fit its registers and LDS.
template <int D, bool F32C> struct BwdShape;
template <> struct BwdShape<32, false> {
  static constexpr int DQ_NW = 4, DQ_QT = 2, DQ_KVS = 64;
  static constexpr int KV_NW = 4, KV_KT = 2, KV_QS = 64;
};
template <> struct BwdShape<32, true> {
  static constexpr int DQ_NW = 4, DQ_QT = 2, DQ_KVS = 64;
  static constexpr int KV_NW = 4, KV_KT = 2, KV_QS = 64;
};
template <> struct BwdShape<64, false> {
  static constexpr int DQ_NW = 8, DQ_QT = 2, DQ_KVS = 64;
  static constexpr int KV_NW = 8, KV_KT = 2, KV_QS = 64;
};
template <> struct BwdShape<64, true> {
  static constexpr int DQ_NW = 4, DQ_QT = 2, DQ_KVS = 64;
  static constexpr int KV_NW = 4, KV_KT = 2, KV_QS = 64;
};
template <> struct BwdShape<128, false> {
  static constexpr int DQ_NW = 8, DQ_QT = 2, DQ_KVS = 64;
  static constexpr int KV_NW = 8, KV_KT = 1, KV_QS = 64;
};
template <> struct BwdShape<128, true> {
  static constexpr int DQ_NW = 8, DQ_QT = 1, DQ_KVS = 64;
  static constexpr int KV_NW = 8, KV_KT = 1, KV_QS = 64;
};
// D = 256: one wave per SIMD (4-wave workgroups), so each wave may hold up to
// 512 registers (VGPRs plus AGPRs): the dK / dV accumulators alone are 128
// per wave.  32-row stages keep the prefetch registers and the fp32 tiles
// (with their transposed copies) within registers and LDS.
template <> struct BwdShape<256, false> {
  static constexpr int DQ_NW = 4, DQ_QT = 1, DQ_KVS = 32;
  static constexpr int KV_NW = 4, KV_KT = 1, KV_QS = 32;
};
template <> struct BwdShape<256, true> {
  static constexpr int DQ_NW = 4, DQ_QT = 1, DQ_KVS = 32;
  static constexpr int KV_NW = 4, KV_KT = 1, KV_QS = 32;
};

template <int D, bool F32C> static int dq_rows() { return BwdShape<D, F32C>::DQ_NW * BwdShape<D, F32C>::DQ_QT * 16; }
template <int D, bool F32C> static int kv_rows() { return BwdShape<D, F32C>::KV_NW * BwdShape<D, F32C>::KV_KT * 16; }
int bwd_dq_block_rows(int D, int ct) {
  const bool f = ct == DT_F32;
  switch (D) {
    case 32: return f ? dq_rows<32, true>() : dq_rows<32, false>();
    case 64: return f ? dq_rows<64, true>() : dq_rows<64, false>();
    case 128: return f ? dq_rows<128, true>() : dq_rows<128, false>();
    default: return f ? dq_rows<256, true>() : dq_rows<256, false>();
  }
}
int bwd_dkdv_block_rows(int D, int ct) {
  const bool f = ct == DT_F32;
  switch (D) {
    case 32: return f ? kv_rows<32, true>() : kv_rows<32, false>();
    case 64: return f ? kv_rows<64, true>() : kv_rows<64, false>();
    case 128: return f ? kv_rows<128, true>() : kv_rows<128, false>();
    default: return f ? kv_rows<256, true>() : kv_rows<256, false>();
  }
}
int bwd_dkdv_threads(int D, int ct) {
  const bool f = ct == DT_F32;
  switch (D) {
    case 32: return 64 * (f ? BwdShape<32, true>::KV_NW : BwdShape<32, false>::KV_NW);
    case 64: return 64 * (f ? BwdShape<64, true>::KV_NW : BwdShape<64, false>::KV_NW);
    case 128: return 64 * (f ? BwdShape<128, true>::KV_NW : BwdShape<128, false>::KV_NW);
    default: return 64 * (f ? BwdShape<256, true>::KV_NW : BwdShape<256, false>::KV_NW);
  }
}

template <typename IO, int D>
static hipError_t pre_io(const BwdParams& p, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8);
  const int64_t total = (int64_t)p.B * p.H * p.N;
  const int grid = (int)((total + RPB - 1) / RPB);
  hipLaunchKernelGGL((bwd_pre_kernel<IO, D>), dim3(grid), dim3(256), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_bwd_pre(const BwdParams& p, int io, int D, hipStream_t st) {
  if (D == 32) {
    switch (io) {
      case DT_BF16: return pre_io<bf16, 32>(p, st);
      case DT_F16: return pre_io<f16, 32>(p, st);
      default: return pre_io<float, 32>(p, st);
    }
  }
  if (D == 64) {
    switch (io) {
      case DT_BF16: return pre_io<bf16, 64>(p, st);
      case DT_F16: return pre_io<f16, 64>(p, st);
      default: return pre_io<float, 64>(p, st);
    }
  }
  if (D == 128) {
    switch (io) {
      case DT_BF16: return pre_io<bf16, 128>(p, st);
      case DT_F16: return pre_io<f16, 128>(p, st);
      default: return pre_io<float, 128>(p, st);
    }
  }
  switch (io) {
    case DT_BF16: return pre_io<bf16, 256>(p, st);
    case DT_F16: return pre_io<f16, 256>(p, st);
    default: return pre_io<float, 256>(p, st);
  }
}

bool bwd_folds_tail(int io, int ct, int D, bool vec) {
  // the XR instantiations of the dQ kernel: 16-bit I/O, fp16 logits, 8 keys
  // per wave and block (D = 128, 256)
  return io != DT_F32 && f16_logits(ct, D) && vec && (D == 128 || D == 256);
}

template <typename IO, int CT, int D>
static hipError_t dq_launch(const BwdParams& p0, bool write_delta, hipStream_t st) {
  using SH = BwdShape<D, CT == DT_F32>;
  constexpr bool FS = f16_logits(CT, D);
  BwdParams p = p0;
  const int grid = p.n_wg = p.B * p.H * p.n_blk;
  // (fp32 compute has no registers to spare for the prefetch)
  if constexpr (CT != DT_F32) {
    if (p.vec_k && p.vec_v) {
      if (write_delta)
        hipLaunchKernelGGL((bwd_dq_kernel<IO, CT, D, SH::DQ_NW, SH::DQ_QT, SH::DQ_KVS, true, true, FS>),
                           dim3(grid), dim3(SH::DQ_NW * 64), 0, st, p);
      else
        hipLaunchKernelGGL((bwd_dq_kernel<IO, CT, D, SH::DQ_NW, SH::DQ_QT, SH::DQ_KVS, false, true, FS>),
                           dim3(grid), dim3(SH::DQ_NW * 64), 0, st, p);
      return hipGetLastError();
    }
  }
  if (write_delta)
    hipLaunchKernelGGL((bwd_dq_kernel<IO, CT, D, SH::DQ_NW, SH::DQ_QT, SH::DQ_KVS, true, false, FS>),
                       dim3(grid), dim3(SH::DQ_NW * 64), 0, st, p);
  else
    hipLaunchKernelGGL((bwd_dq_kernel<IO, CT, D, SH::DQ_NW, SH::DQ_QT, SH::DQ_KVS, false, false, FS>),
                       dim3(grid), dim3(SH::DQ_NW * 64), 0, st, p);
  return hipGetLastError();
}

template <typename IO, int CT, int D>
static hipError_t dkdv_launch(const BwdParams& p0, hipStream_t st) {
  using SH = BwdShape<D, CT == DT_F32>;
  constexpr bool FS = f16_logits(CT, D);
  BwdParams p = p0;
  const int grid = p.n_wg = p.B * p.H * p.n_blk;
  // (fp32 compute has no registers to spare for the prefetch)
  if constexpr (CT != DT_F32) {
    if (p.vec_q && p.vec_do) {
      if constexpr (FS) {
        if (p.qhat_f) {
          hipLaunchKernelGGL((bwd_dkdv_kernel<IO, CT, D, SH::KV_NW, SH::KV_KT, SH::KV_QS, true, FS, true>),
                             dim3(grid), dim3(SH::KV_NW * 64), 0, st, p);
          return hipGetLastError();
        }
      }
      hipLaunchKernelGGL((bwd_dkdv_kernel<IO, CT, D, SH::KV_NW, SH::KV_KT, SH::KV_QS, true, FS, false>), dim3(grid),
                         dim3(SH::KV_NW * 64), 0, st, p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((bwd_dkdv_kernel<IO, CT, D, SH::KV_NW, SH::KV_KT, SH::KV_QS, false, FS, false>), dim3(grid),
                     dim3(SH::KV_NW * 64), 0, st, p);
  return hipGetLastError();
}

template <typename IO, int D>
static hipError_t dq_ct(const BwdParams& p, int ct, bool wd, hipStream_t st) {
  switch (ct) {
    case DT_BF16: return dq_launch<IO, DT_BF16, D>(p, wd, st);
    case DT_F16: return dq_launch<IO, DT_F16, D>(p, wd, st);
    default: return dq_launch<IO, DT_F32, D>(p, wd, st);
  }
}
template <int D>
static hipError_t dq_io(const BwdParams& p, int io, int ct, bool wd, hipStream_t st) {
  switch (io) {
    case DT_BF16: return dq_ct<bf16, D>(p, ct, wd, st);
    case DT_F16: return dq_ct<f16, D>(p, ct, wd, st);
    default: return dq_ct<float, D>(p, ct, wd, st);
  }
}
hipError_t launch_bwd_dq(const BwdParams& p, int io, int ct, int D, bool write_delta,
                         hipStream_t st) {
  switch (D) {
    case 32: return dq_io<32>(p, io, ct, write_delta, st);
    case 64: return dq_io<64>(p, io, ct, write_delta, st);
    case 128: return dq_io<128>(p, io, ct, write_delta, st);
    default: return dq_io<256>(p, io, ct, write_delta, st);
  }
}

template <typename IO, int D>
static hipError_t kv_ct(const BwdParams& p, int ct, hipStream_t st) {
  switch (ct) {
    case DT_BF16: return dkdv_launch<IO, DT_BF16, D>(p, st);
    case DT_F16: return dkdv_launch<IO, DT_F16, D>(p, st);
    default: return dkdv_launch<IO, DT_F32, D>(p, st);
  }
}
template <int D>
static hipError_t kv_io(const BwdParams& p, int io, int ct, hipStream_t st) {
  switch (io) {
    case DT_BF16: return kv_ct<bf16, D>(p, ct, st);
    case DT_F16: return kv_ct<f16, D>(p, ct, st);
    default: return kv_ct<float, D>(p, ct, st);
  }
}
hipError_t launch_bwd_dkdv(const BwdParams& p, int io, int ct, int D, hipStream_t st) {
  switch (D) {
    case 32: return kv_io<32>(p, io, ct, st);
    case 64: return kv_io<64>(p, io, ct, st);
    case 128: return kv_io<128>(p, io, ct, st);
    default: return kv_io<256>(p, io, ct, st);
  }
}

// ---------------------------------------------------------------------------
// Packed RoPE table: out[0] = identity row, out[l + 1][p] = (cos, sin).
// ---------------------------------------------------------------------------
__global__ void rope_pack_kernel(const float* __restrict__ cosp, int64_t cs0, int64_t cs1,
                                 const float* __restrict__ sinp, int64_t ss0, int64_t ss1,
                                 int n_pos, int d2, float* __restrict__ out) {
  const int64_t i = (int64_t)block_id() * 256 + thread_id();
  const int64_t total = (int64_t)(n_pos + 1) * d2;
  if (i >= total) return;
  const int row = (int)(i / d2), pr = (int)(i - (int64_t)row * d2);
  float c = 1.f, s = 0.f;
  if (row > 0) {
    c = cosp[(int64_t)(row - 1) * cs0 + pr * cs1];
    s = sinp[(int64_t)(row - 1) * ss0 + pr * ss1];
  }
  out[2 * i] = c;
  out[2 * i + 1] = s;
}

hipError_t launch_rope_pack(const float* cosp, int64_t cs0, int64_t cs1, const float* sinp,
                            int64_t ss0, int64_t ss1, int n_pos, int d2, float* out,
                            hipStream_t st) {
  const int64_t total = (int64_t)(n_pos + 1) * d2;
  const int grid = (int)((total + 255) / 256);
  hipLaunchKernelGGL(rope_pack_kernel, dim3(grid), dim3(256), 0, st, cosp, cs0, cs1, sinp, ss0,
                     ss1, n_pos, d2, out);
  return hipGetLastError();
}

}  // namespace farope
