// Stored-dS backward for the key-tile shapes (16-bit I/O, bf16 compute,
// head_dim 128, vector access to every tensor): the key tiles (bwd_keys.hip)
// keep the dS they form, and dQ becomes one GEMM over it, so S and dP are
// computed once per (query, key) instead of once per pass.
//
// Reference behaviour followed ("fa_rope_full .py"):
//   delta = rowsum(dO * O) in fp32                      _attn_bwd_preprocess FA:325-357
//   dQ-hat = dS K-hat, dQ = R^T dQ-hat * scale          _attn_bwd_dq_rope    FA:708-1009
//   the lone last key's dK / dV: as the key tiles       _attn_bwd_dk_dv_rope FA:374-691
// with the CLS row bypassing the rotation (FA:647-662, FA:980-993).
//
// Order of one backward: bwd_ds_prep_kernel (per 64-row tile: delta, the
// fp16 rows Q-hat * c2 (c2 = scale * log2 e) and the row statistics the key
// tiles stage; with one key past the full key tiles, that key's dS per row and
// the tile's partial dK-hat / dV rows), the key tiles (dK, dV; they store
// sig dS^T and K-hat * fk in fp16 with each tile's exponent of 1 / (sig fk)),
// then bwd_ds_dq_kernel (dQ; the first tile of each plane also adds up the
// last key's partial rows into its dK / dV).
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

namespace {
constexpr int kDsD = 128;
constexpr int kCachePolicyNT = 2;   // buffer instruction cache-policy bit nt (gfx950)

template <typename IO>
__device__ __forceinline__ const IO* plane_ptr(const void* b, const int64_t* st, int plane, int H) {
  const int bb = plane / H, hh = plane - bb * H;
  return static_cast<const IO*>(b) + bb * st[0] + hh * st[1];
}

// sum / max over each aligned group of 16 lanes (one 16-lane DPP row)
__device__ __forceinline__ float sum16(float x) {
  x = dpp_sum8(x);
  return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));   // row_ror:8
}
__device__ __forceinline__ float max16(float x) {
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false)));
  x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false)));
  return fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false)));
}
}  // namespace

// ---------------------------------------------------------------------------
// Row pass.  One 256-thread workgroup per (plane, 64-row tile); 16 lanes per
// row (8 channels each), 4 rows per wave and step, 4 steps.
// ---------------------------------------------------------------------------
template <typename IO>
__global__ void __launch_bounds__(256) bwd_ds_prep_kernel(const BwdParams p, int n_pt) {
  constexpr int D = kDsD, D2 = D / 2, RT = kDsPrepRows;
  __shared__ __attribute__((aligned(16))) float sX[4][2 * D];
  const int N = p.N;
  const int tile = block_id();
  const int plane = tile / n_pt, pt = tile - plane * n_pt;
  const IO* __restrict__ Q = plane_ptr<IO>(p.q, p.sq, plane, p.H);
  const IO* __restrict__ O = plane_ptr<IO>(p.o, p.so, plane, p.H);
  const IO* __restrict__ G = plane_ptr<IO>(p.dout, p.sdo, plane, p.H);
  const float* __restrict__ tab = p.rope;
  const int shift = 1 - p.has_cls;
  const int64_t prow = (int64_t)plane * N;
  const float c2 = p.scale_log2;
  const int tid = thread_id(), wave = tid >> 6, lane = tid & 63;
  const int cc = lane & 15, c0 = 8 * cc, rsub = lane >> 4;
  const bool last = p.dslast != nullptr;

  // every step's rows are loaded first (buffer descriptors over the plane:
  // rows >= N read zeros; without a residual its range is empty), so all of
  // the tile's loads are in flight at once (a branch around any of them would
  // make the compiler wait for all of them there)
  constexpr int ST = RT / 16;
  const unsigned ES = sizeof(IO);
  const auto rQ = make_rsrc(Q, (unsigned)(((int64_t)(N - 1) * p.sq[2] + D) * ES));
  const auto rG = make_rsrc(G, (unsigned)(((int64_t)(N - 1) * p.sdo[2] + D) * ES));
  const auto rO = make_rsrc(O, (unsigned)(((int64_t)(N - 1) * p.so[2] + D) * ES));
  const auto rR = make_rsrc(p.o_res ? static_cast<const IO*>(p.o_res) + prow * D : nullptr,
                            p.o_res ? (unsigned)(N * D * ES) : 0u);
  const auto rL = make_rsrc(p.lse + prow, (unsigned)N * 4u);
  Raw8<IO> rq[ST], rg[ST], ro[ST], rr[ST], rkl, rvl;
  float cs[ST][8], lsv[ST], ckl[8];
  rkl = load_raw8(plane_ptr<IO>(p.k, p.sk, plane, p.H) + (int64_t)(N - 1) * p.sk[2] + c0, 1, true);
  rvl = load_raw8(plane_ptr<IO>(p.v, p.sv, plane, p.H) + (int64_t)(N - 1) * p.sv[2] + c0, 1, true);
  rope_load4(tab, N - 1 + shift, D2, 4 * cc, ckl);
  __builtin_amdgcn_sched_barrier(0);   // (keeps them ahead of the row loads)
#pragma unroll
  for (int it = 0; it < ST; ++it) {
    const int r = pt * RT + it * 16 + wave * 4 + rsub;
    rq[it] = buf_load8<IO>(rQ, (unsigned)((r * (int)p.sq[2] + c0) * (int)ES), 0u);
    rg[it] = buf_load8<IO>(rG, (unsigned)((r * (int)p.sdo[2] + c0) * (int)ES), 0u);
    ro[it] = buf_load8<IO>(rO, (unsigned)((r * (int)p.so[2] + c0) * (int)ES), 0u);
    rr[it] = buf_load8<IO>(rR, (unsigned)((r * D + c0) * (int)ES), 0u);
    rope_load4(tab, min(r, N - 1) + shift, D2, 4 * cc, cs[it]);
    lsv[it] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rL, (unsigned)r * 4u, 0u, 0));
  }
  // the last key's K-hat (logit units: the rows below carry c2) and V
  // channels (row N - 1 is loaded either way, first: the global loads complete
  // in order; used with p.dslast only)
  float kl[8], vl[8];
  unpack8(rkl, kl);
  rope_rotate8(kl, ckl);
  unpack8(rvl, vl);
  float xk[8] = {}, xv[8] = {};
#pragma unroll
  for (int it = 0; it < ST; ++it) {
    const int r = pt * RT + it * 16 + wave * 4 + rsub;
    const bool ok = r < N;
    float x[8], g[8], o[8], xs[8];
    float dsum = 0.f, gn2 = 0.f, s = 0.f, dp = 0.f;
    unpack8(rq[it], x);
    rope_rotate8(x, cs[it]);
    unpack8(rg[it], g);
    unpack8(ro[it], o);
#pragma unroll
    for (int e = 0; e < 8; ++e) dsum += g[e] * o[e];
    unpack8(rr[it], o);   // O's rounding residual (contiguous [B, H, N, D]), or zeros
#pragma unroll
    for (int e = 0; e < 8; ++e) dsum += g[e] * o[e];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xs[e] = x[e] * c2;
      gn2 = __builtin_fmaf(g[e], g[e], gn2);
    }
    float qm = amax8(0.f, xs);
    if (ok) *reinterpret_cast<f16x8*>(static_cast<f16*>(p.qhat_f) + (prow + r) * D + c0) = to_f16x8(xs);
    if (last) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s = __builtin_fmaf(xs[e], kl[e], s);
        dp = __builtin_fmaf(g[e], vl[e], dp);
      }
    }
    dsum = sum16(dsum);
    gn2 = sum16(gn2);
    qm = max16(qm);
    if (ok && cc == 0) {
      p.delta[prow + r] = dsum;
      reinterpret_cast<float2*>(p.row_stat)[prow + r] = make_float2(__builtin_sqrtf(gn2), qm);
    }
    if (last) {
      s = sum16(s);
      dp = sum16(dp);
      float pr = 0.f, ds = 0.f;
      if (ok) {
        pr = __builtin_amdgcn_fmed3f(fast_exp2(s - lsv[it] * kLog2e), 0.f, 1.f);
        ds = pr * (dp - dsum);
        if (cc == 0) p.dslast[prow + r] = ds;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {   // (x, g are zero past row N - 1)
        xk[e] = __builtin_fmaf(ds, x[e], xk[e]);
        xv[e] = __builtin_fmaf(pr, g[e], xv[e]);
      }
    }
  }
  if (last) {
    // the tile's partial rows of the last key: dK-hat (without scale) and dV
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xk[e] = group4_sum(xk[e]);
      xv[e] = group4_sum(xv[e]);
    }
    if (rsub == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sX[wave][c0 + e] = xk[e];
        sX[wave][D + c0 + e] = xv[e];
      }
    }
    lds_barrier();
    p.xk_ws[((int64_t)plane * n_pt + pt) * (2 * D) + tid] = sX[0][tid] + sX[1][tid] + sX[2][tid] + sX[3][tid];
  }
}

// ---------------------------------------------------------------------------
// dQ GEMM.  One 8-wave workgroup per (plane, 256-query tile).  Key tile t
// stored (sig_t dS^T) and (K-hat fk_t) in fp16, with e_t = log2 of
// 1 / (sig_t fk_t); with e_max the plane's largest e_t,
//   dQ-hat^T[c][q] = 2^e_max * sum_t sum_{k in t}
//                    (2^(e_t - e_max) K-hat fk_t)[k][c] (sig_t dS^T)[k][q]
// so each tile's K-hat rows are staged times 2^(e_t - e_max) (an exact power
// of two <= 1; a tile more than 2^24 below the largest drops out) and one
// fp32 accumulator serves every tile.  The lone last key adds
// dS[q] K-hat[c] in fp32 at the end.
// Wave w covers channels 64 (w / 4) .. and queries 64 (w % 4) .. of the tile
// (4 x 4 MFMA blocks); blocks of 64 keys are staged in LDS (dS^T [64][256 + 8],
// K-hat [64][128 + 8], rows padded by 16 bytes) from registers loaded two
// blocks ahead, and both operands are read transposed (ds_read_b64_tr_b16).
// ---------------------------------------------------------------------------
template <typename IO, int QR, int NW>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
bwd_ds_dq_kernel(const BwdParams p, int n_qt) {
  using H = Comp<DT_F16>;
  using HFrag = H::Frag;
  constexpr int D = kDsD, D2 = D / 2, KB = 64, NT = NW * 64;
  constexpr int WQ = QR / 64;   // waves along the queries (64 each); NW / WQ along the channels
  static_assert(WQ * (D / 64) == NW, "wave tiling: 64 x 64 per wave");
  constexpr int LDS_ = QR + 8, LDK = D + 8;
  constexpr int SI = KB * QR / 8 / NT, KI = KB * D / 8 / NT;   // 16-byte units per thread
  static_assert(SI * NT * 8 == KB * QR && KI * NT * 8 == KB * D && kKeysRows % KB == 0, "tile shape");
  __shared__ __attribute__((aligned(16))) f16 sS[2][KB * LDS_];
  __shared__ __attribute__((aligned(16))) f16 sK[2][KB * LDK];
  __shared__ f16 sF[kDsMaxKeyTiles];   // per key tile: 2^(e_t - e_max)

  const int N = p.N, n_kt = p.n_kt, KP = n_kt * kKeysRows, NQP = p.nqp;
  const int tile = xcd_remap(block_id(), p.n_wg);
  const int plane = tile / n_qt, qt = tile - plane * n_qt;
  const int q0 = qt * QR;
  const int tid = thread_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, lr = lane & 15, lg = lane >> 4;
  const int qw = 64 * (wave % WQ), cw = 64 * (wave / WQ);

  const int* __restrict__ kexp = p.kexp + (int64_t)plane * n_kt;
  int emax = kexp[0];
  for (int t = 1; t < n_kt; ++t) emax = max(emax, kexp[t]);
  emax = __builtin_amdgcn_readfirstlane(emax);
  // (in LDS: a global load in the loop would be waited for behind the block loads)
  for (int t = tid; t < n_kt; t += NT) sF[t] = (f16)__builtin_ldexpf(1.f, kexp[t] - emax);   // 0 below fp16's range
  lds_barrier();

  const auto rS = make_rsrc(static_cast<const f16*>(p.ds_t) + (int64_t)plane * KP * NQP, (unsigned)(KP * NQP * 2));
  const auto rK = make_rsrc(static_cast<const f16*>(p.khat) + (int64_t)plane * KP * D, (unsigned)(KP * D * 2));
  // staging units: dS^T row sr + 16 i, queries q0 + 8 sc ..; K-hat row kr + 32 i, channels 8 kc ..
  // (the key tiles write the columns below N rounded up to 32, zeros past N;
  // later ones are staged as zeros: their lane offset is past the range)
  constexpr int SC = QR / 8, SR = NT / SC, KR = NT / 16;   // 16-byte units per dS^T row; rows per pass
  const int sr = tid / SC, sc = tid % SC, kr = tid >> 4, kc = tid & 15;
  const unsigned svo = q0 + 8 * sc < round_up32(N) ? (unsigned)((sr * NQP + q0 + 8 * sc) * 2) : 0x80000000u;
  const unsigned kvo = (unsigned)((kr * D + 8 * kc) * 2);
  u32x4 ps[2][SI], pk[2][KI];
  auto load = [&](auto setc, int kb) __attribute__((always_inline)) {
    constexpr int s = decltype(setc)::value;
    // past the last block: offsets beyond the range, zeros (never committed).
    // dS^T is read once: non-temporal loads (cache policy nt), so it does not
    // displace the K-hat rows the plane's other query tiles re-read from L2
    const unsigned bs = (unsigned)(kb * KB * NQP * 2), bk = (unsigned)(kb * KB * D * 2);
#pragma unroll
    for (int i = 0; i < SI; ++i)
      ps[s][i] = __builtin_amdgcn_raw_buffer_load_b128(rS, svo + (unsigned)(i * SR * NQP * 2), bs, kCachePolicyNT);
#pragma unroll
    for (int i = 0; i < KI; ++i)
      pk[s][i] = __builtin_amdgcn_raw_buffer_load_b128(rK, kvo + (unsigned)(i * KR * D * 2), bk, 0);
  };
  auto commit = [&](auto setc, auto bufc, int kb) __attribute__((always_inline)) {
    constexpr int s = decltype(setc)::value, b = decltype(bufc)::value;
#pragma unroll
    for (int i = 0; i < SI; ++i) *reinterpret_cast<u32x4*>(&sS[b][(sr + SR * i) * LDS_ + 8 * sc]) = ps[s][i];
    // this tile's K-hat rows to the plane's exponent (unconditionally: a
    // branch here makes the compiler wait for every load in flight)
    const f16 f = sF[min(kb / (kKeysRows / KB), n_kt - 1)];
#pragma unroll
    for (int i = 0; i < KI; ++i) {
      f16x8 h = __builtin_bit_cast(f16x8, pk[s][i]);
      h = h * f;
      pk[s][i] = __builtin_bit_cast(u32x4, h);
    }
#pragma unroll
    for (int i = 0; i < KI; ++i) *reinterpret_cast<u32x4*>(&sK[b][(kr + KR * i) * LDK + 8 * kc]) = pk[s][i];
  };

  f32x4 acc[4][4];   // [channel block][query block]
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  // query blocks of the wave inside the plane (4 except in a ragged last tile)
  const int nq = min(4, max(0, (N - q0 - qw + 15) / 16));

  auto compute = [&](auto bufc, auto fullc) __attribute__((always_inline)) {
    constexpr int b = decltype(bufc)::value;
    constexpr bool full = decltype(fullc)::value;
#pragma unroll
    for (int ks = 0; ks < KB / 32; ++ks) {
      const int r0 = 32 * ks + 8 * lg + (lr >> 2);
      HFrag a[4], q[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int ck = cw + 16 * t + 4 * (lr & 3), cq = qw + 16 * t + 4 * (lr & 3);
        a[t] = H::tr(&sK[b][r0 * LDK + ck], &sK[b][(r0 + 4) * LDK + ck]);
        q[t] = H::tr(&sS[b][r0 * LDS_ + cq], &sS[b][(r0 + 4) * LDS_ + cq]);
      }
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (full || u < nq) acc[t][u] = H::mma(a[t], q[u], acc[t][u]);
    }
  };
  // Blocks kb (buffer 0) and kb + 1 (buffer 1) per trip; the registers hold
  // the two blocks after the committed one.
  auto run = [&](auto fullc) __attribute__((always_inline)) {
    const int nkb = KP / KB;   // even
    load(std::integral_constant<int, 0>{}, 0);
    load(std::integral_constant<int, 1>{}, 1);
    commit(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, 0);
    load(std::integral_constant<int, 0>{}, 2);
    for (int kb = 0; kb < nkb; kb += 2) {
      lds_barrier();
      compute(std::integral_constant<int, 0>{}, fullc);
      commit(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, kb + 1);
      load(std::integral_constant<int, 1>{}, kb + 3);
      lds_barrier();
      compute(std::integral_constant<int, 1>{}, fullc);
      // (also past the last block, where the rows are zeros that are never
      // read: a branch here makes the compiler wait for every load in flight)
      commit(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, kb + 2);
      load(std::integral_constant<int, 0>{}, kb + 4);
    }
  };
  if (q0 + QR <= N)
    run(std::true_type{});
  else
    run(std::false_type{});

  // ---- epilogue: lane holds dQ-hat^T of channels cw + 16t + 4lg + (0..3), query qw + 16u + lr ----
  const int shift = 1 - p.has_cls;
  const int64_t prow = (int64_t)plane * N;
  const float* __restrict__ tab = p.rope;
  IO* __restrict__ dQ = const_cast<IO*>(plane_ptr<IO>(p.dq, p.sdq, plane, p.H));
  float kl[4][4] = {};   // the lone last key's K-hat at the lane's channels (fp32)
  if (p.dslast) {
    const IO* K = plane_ptr<IO>(p.k, p.sk, plane, p.H) + (int64_t)(N - 1) * p.sk[2];
    typedef IO io4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int c = cw + 16 * t + 4 * lg;
      const io4 kv = *reinterpret_cast<const io4*>(K + c);
      const f32x4 cs = *reinterpret_cast<const f32x4*>(tab + ((int64_t)(N - 1 + shift) * D2 + c / 2) * 2);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const float e = (float)kv[2 * h], o = (float)kv[2 * h + 1];
        kl[t][2 * h] = e * cs[2 * h] - o * cs[2 * h + 1];
        kl[t][2 * h + 1] = o * cs[2 * h] + e * cs[2 * h + 1];
      }
    }
  }
  // 16 bytes per lane and store: lane groups lg and lg^1 trade halves
  // (v_permlane16_swap), even lg then holding channels cw + 16 t0 + 4 lg .. + 7
  // and odd lg channels cw + 16 (t0 + 1) + 4 (lg - 1) .. + 7; half the store
  // instructions of 8-byte stores.  Every lane takes part in the exchange:
  // queries >= N (their products were skipped or hold zero rows) fall
  // outside the descriptor's range, and their table row and dS of the last
  // key are clamped to query N - 1.
  {
    const auto rQ = make_rsrc(dQ, (unsigned)(((int64_t)(N - 1) * p.sdq[2] + D) * sizeof(IO)));
    typedef IO io4 __attribute__((ext_vector_type(4)));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int q = q0 + qw + 16 * u + lr;
      const int qc = min(q, N - 1);
      const float dl = p.dslast ? p.dslast[prow + qc] : 0.f;
#pragma unroll
      for (int t0 = 0; t0 < 4; t0 += 2) {
        u32x2 w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int t = t0 + h;
          const int c = cw + 16 * t + 4 * lg;
          float g4[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            g4[i] = p.scale * __builtin_fmaf(dl, kl[t][i], __builtin_ldexpf(acc[t][u][i], emax));
          rope_unrotate4(g4, tab, qc + shift, D2, c / 2);
          io4 a;
#pragma unroll
          for (int i = 0; i < 4; ++i) a[i] = (IO)g4[i];
          __builtin_memcpy(&w[h], &a, 8);
        }
        u32x4 x;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto r = __builtin_amdgcn_permlane16_swap(w[0][k], w[1][k], false, false);
          x[k] = r[0];
          x[2 + k] = r[1];
        }
        const int ch = cw + 16 * (t0 + (lg & 1)) + 4 * (lg & 2);
        buf_store16(x, rQ, (unsigned)((q * (int)p.sdq[2] + ch) * (int)sizeof(IO)), 0u);
      }
    }
  }
  // the lone last key's dK / dV (the plane's first tile): the row pass's
  // partial rows added in order, dK-hat scaled and rotated back
  if (p.dslast && qt == 0 && tid < D / 4) {
    const int n_pt = (N + kDsPrepRows - 1) / kDsPrepRows, kc = N - 1;
    const float* w = p.xk_ws + (int64_t)plane * n_pt * (2 * D);
    float xk[4] = {}, xv[4] = {};
    for (int b = 0; b < n_pt; ++b) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(w + b * 2 * D + 4 * tid);
      const f32x4 v = *reinterpret_cast<const f32x4*>(w + b * 2 * D + D + 4 * tid);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xk[e] += a[e];
        xv[e] += v[e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) xk[e] *= p.scale;
    rope_unrotate4(xk, tab, kc + shift, D2, 2 * tid);
    IO* DK = const_cast<IO*>(plane_ptr<IO>(p.dk, p.sdk, plane, p.H)) + (int64_t)kc * p.sdk[2];
    IO* DV = const_cast<IO*>(plane_ptr<IO>(p.dv, p.sdv, plane, p.H)) + (int64_t)kc * p.sdv[2];
    store4(DK + 4 * tid, 1, true, xk);
    store4(DV + 4 * tid, 1, true, xv);
  }
}

hipError_t launch_bwd_ds_prep(const BwdParams& p, int io, hipStream_t st) {
  const int n_pt = (p.N + kDsPrepRows - 1) / kDsPrepRows;
  const dim3 grid(p.B * p.H * n_pt);
  switch (io) {
    case DT_BF16: hipLaunchKernelGGL((bwd_ds_prep_kernel<bf16>), grid, dim3(256), 0, st, p, n_pt); break;
    case DT_F16: hipLaunchKernelGGL((bwd_ds_prep_kernel<f16>), grid, dim3(256), 0, st, p, n_pt); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_ds_dq(const BwdParams& p0, int io, hipStream_t st) {
  BwdParams p = p0;
  constexpr int QR = kDsQueryRows, NW = QR / 64 * 2;
  const int n_qt = (p.N + QR - 1) / QR;
  p.n_wg = p.B * p.H * n_qt;
  switch (io) {
    case DT_BF16: hipLaunchKernelGGL((bwd_ds_dq_kernel<bf16, QR, NW>), dim3(p.n_wg), dim3(NW * 64), 0, st, p, n_qt); break;
    case DT_F16: hipLaunchKernelGGL((bwd_ds_dq_kernel<f16, QR, NW>), dim3(p.n_wg), dim3(NW * 64), 0, st, p, n_qt); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace farope
