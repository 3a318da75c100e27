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
// Workgroup = NW waves.  Wave w owns key subtiles w, w+NW, ... (16 keys
// each): their K-hat and V rows sit in registers as MFMA B-operands, their
// dK-hat / dV accumulators in registers.  The plane's queries are swept in
// stages of QS rows:
//   commit   staged registers -> LDS: Q-hat and dO row-major (rows permuted
//            so one MFMA's 16 A-rows are consecutive), Q-hat^T and dO^T
//            (two rows per 32-bit write), LSE*log2(e), delta = rowsum(dO*O)
//   prefetch the next stage's Q, dO, O, LSE rows into registers
//   barrier
//   S, dP for each owned key subtile (query rows permuted so lane group lg
//            holds queries 8lg..8lg+7: P and dS land in the B-operand layout
//            of dV^T += dO^T P and dK-hat^T += Q-hat^T dS); dS -> LDS
//   barrier
//   dQ-hat^T = K-hat^T dS^T for the stage's rows (K-hat^T of the whole
//            plane was staged once), un-rotate, store.
// Q, K, V, O, dO are read from HBM once; dQ, dK, dV written once.
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

template <int CT> __device__ __forceinline__ void put2b(typename Comp<CT>::S* p, float a, float b);
template <> __device__ __forceinline__ void put2b<DT_BF16>(bf16* p, float a, float b) {
  typedef bf16 v2 __attribute__((ext_vector_type(2)));
  v2 v;
  v[0] = (bf16)a;
  v[1] = (bf16)b;
  *reinterpret_cast<v2*>(p) = v;
}
template <> __device__ __forceinline__ void put2b<DT_F16>(f16* p, float a, float b) {
  typedef f16 v2 __attribute__((ext_vector_type(2)));
  v2 v;
  v[0] = (f16)a;
  v[1] = (f16)b;
  *reinterpret_cast<v2*>(p) = v;
}
template <> __device__ __forceinline__ void put2b<DT_F32>(float* p, float a, float b) {
  typedef float v2 __attribute__((ext_vector_type(2)));
  v2 v;
  v[0] = a;
  v[1] = b;
  *reinterpret_cast<v2*>(p) = v;
}

// Within each 32-row block, row r = 8a + 4h + i is stored at 16h + 4a + i.
__device__ __forceinline__ int rperm(int r) {
  return (r & ~31) | ((r & 4) << 2) | ((r & 24) >> 1) | (r & 3);
}

// VEC: every tensor of the call allows 16-byte vector access (decided on the
// host); the generic instantiation gathers element by element instead.
template <typename IO, int CT, int D, int NW, int KT, int QS, bool VEC>
__global__ void __launch_bounds__(NW * 64)
bwd_fused_kernel(const BwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  constexpr int KS = D / 32, DT = D / 16, D2 = D / 2;
  constexpr int PADE = 16 / sizeof(S);
  constexpr int LDQ = D + PADE;          // row-major Q-hat / dO pitch
  constexpr int LDT = QS + PADE;         // transposed Q-hat^T / dO^T pitch
  constexpr int NT = NW * 64, CPR = D / 8;
  constexpr int KROWS = NW * KT * 16;    // keys per workgroup (>= N)
  constexpr int LDKT = KROWS + PADE;     // K-hat^T and dS pitch
  constexpr int QUNITS = (QS / 2) * CPR; // (row pair, chunk) units of one tensor per stage
  static_assert(QUNITS * 2 == NT, "stage staging assumes one Q unit and one dO unit per thread pair");
  static_assert(KT <= 2, "active-subtile dispatch handles KT <= 2");
  constexpr int KUNITS = (KROWS / 2) * CPR;
  constexpr int KITER = (KUNITS + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) S sQ[QS * LDQ];
  __shared__ __attribute__((aligned(16))) S sQt[D * LDT];
  __shared__ __attribute__((aligned(16))) S sG[QS * LDQ];
  __shared__ __attribute__((aligned(16))) S sGt[D * LDT];
  __shared__ __attribute__((aligned(16))) float sL2[QS];
  __shared__ __attribute__((aligned(16))) float sDl[QS];
  __shared__ __attribute__((aligned(16))) S sKt[D * LDKT];
  __shared__ __attribute__((aligned(16))) S sdS[QS * LDKT];

  const int N = p.N;
  const bool vec_q = VEC || p.vec_q, vec_k = VEC || p.vec_k, vec_v = VEC || p.vec_v;
  const bool vec_o = VEC || p.vec_o, vec_do = VEC || p.vec_do, vec_dq = VEC || p.vec_dq;
  const bool vec_dk = VEC || p.vec_dk, vec_dv = VEC || p.vec_dv;
  const int plane = xcd_remap(blockIdx.x, gridDim.x);
  const int bb = plane / p.H, hh = plane - bb * p.H;
  const IO* __restrict__ Q = static_cast<const IO*>(p.q) + bb * p.sq[0] + hh * p.sq[1];
  const IO* __restrict__ K = static_cast<const IO*>(p.k) + bb * p.sk[0] + hh * p.sk[1];
  const IO* __restrict__ V = static_cast<const IO*>(p.v) + bb * p.sv[0] + hh * p.sv[1];
  const IO* __restrict__ O = static_cast<const IO*>(p.o) + bb * p.so[0] + hh * p.so[1];
  const IO* __restrict__ G = static_cast<const IO*>(p.dout) + bb * p.sdo[0] + hh * p.sdo[1];
  IO* __restrict__ dQ = static_cast<IO*>(p.dq) + bb * p.sdq[0] + hh * p.sdq[1];
  IO* __restrict__ dK = static_cast<IO*>(p.dk) + bb * p.sdk[0] + hh * p.sdk[1];
  IO* __restrict__ dV = static_cast<IO*>(p.dv) + bb * p.sdv[0] + hh * p.sdv[1];
  const float* __restrict__ tab = p.rope;
  const int shift = 1 - p.has_cls;
  const int64_t prow = (int64_t)plane * N;
  const float c2 = p.scale_log2;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // ---- stage prefetch: threads [0, NT/2) carry Q (+ cos/sin), the rest dO and O.
  //      The two roles share one register block: Q | cos/sin  or  dO | O. ----
  constexpr int W = (int)(sizeof(Raw8<IO>) / 4);          // 32-bit words per raw row segment
  constexpr int NPRE = (2 * W + 16 > 4 * W) ? 2 * W + 16 : 4 * W;
  const bool q_thread = tid < QUNITS;
  const int su = q_thread ? tid : tid - QUNITS;
  const int srp = su / CPR, scc = su - srp * CPR;   // row pair, 8-channel chunk
  uint32_t pre[NPRE];
  float rlse = 0.f;
  auto put_raw = [&](int slot, const Raw8<IO>& r) { __builtin_memcpy(&pre[slot * W], &r, sizeof(r)); };
  auto get_raw = [&](int slot) {
    Raw8<IO> r;
    __builtin_memcpy(&r, &pre[slot * W], sizeof(r));
    return r;
  };
  auto prefetch = [&](int qb) {
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int gr = qb + 2 * srp + x;
      if (q_thread) {
        float cs[8];
        if (gr < N) {
          put_raw(x, load_raw8(Q + gr * p.sq[2] + 8 * scc * p.sq[3], p.sq[3], vec_q));
          rope_load4(tab, gr + shift, D2, 4 * scc, cs);
        } else {
          put_raw(x, zero_raw8<IO>());
#pragma unroll
          for (int e = 0; e < 8; ++e) cs[e] = 0.f;
        }
        __builtin_memcpy(&pre[2 * W + 8 * x], cs, sizeof(cs));
      } else {
        if (gr < N) {
          put_raw(x, load_raw8(G + gr * p.sdo[2] + 8 * scc * p.sdo[3], p.sdo[3], vec_do));
          put_raw(2 + x, load_raw8(O + gr * p.so[2] + 8 * scc * p.so[3], p.so[3], vec_o));
        } else {
          put_raw(x, zero_raw8<IO>());
          put_raw(2 + x, zero_raw8<IO>());
        }
      }
    }
    if (tid < QS) rlse = qb + tid < N ? p.lse[prow + qb + tid] * kLog2e : INFINITY;
  };
  auto commit = [&]() {
    float x0[8], x1[8];
    unpack8(get_raw(0), x0);
    unpack8(get_raw(1), x1);
    if (q_thread) {
      float cs0[8], cs1[8];
      __builtin_memcpy(cs0, &pre[2 * W], sizeof(cs0));
      __builtin_memcpy(cs1, &pre[2 * W + 8], sizeof(cs1));
      rope_rotate8(x0, cs0);
      rope_rotate8(x1, cs1);
      C::put8(&sQ[rperm(2 * srp) * LDQ + 8 * scc], x0);
      C::put8(&sQ[rperm(2 * srp + 1) * LDQ + 8 * scc], x1);
#pragma unroll
      for (int e = 0; e < 8; ++e) put2b<CT>(&sQt[(8 * scc + e) * LDT + 2 * srp], x0[e], x1[e]);
    } else {
      C::put8(&sG[rperm(2 * srp) * LDQ + 8 * scc], x0);
      C::put8(&sG[rperm(2 * srp + 1) * LDQ + 8 * scc], x1);
#pragma unroll
      for (int e = 0; e < 8; ++e) put2b<CT>(&sGt[(8 * scc + e) * LDT + 2 * srp], x0[e], x1[e]);
      float o0[8], o1[8];
      unpack8(get_raw(2), o0);
      unpack8(get_raw(3), o1);
      float d0 = 0.f, d1 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d0 += x0[e] * o0[e];
        d1 += x1[e] * o1[e];
      }
      // the CPR chunks of a row pair are CPR consecutive lanes of one wave
#pragma unroll
      for (int m = 1; m < CPR; m <<= 1) {
        d0 += __shfl_xor(d0, m);
        d1 += __shfl_xor(d1, m);
      }
      if (scc == 0) {
        sDl[2 * srp] = d0;
        sDl[2 * srp + 1] = d1;
      }
    }
    if (tid < QS) sL2[tid] = rlse;
  };

  prefetch(0);

  // ---- own key subtiles: K-hat and V rows as B-operands ----
  Frag kf[KT][KS], vf[KT][KS];
  int nu = 0;   // owned subtiles holding keys < N: a prefix u < nu (wave-uniform)
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    const int kv0 = (u * NW + wave) * 16;
    nu += kv0 < N;
    const int row = kv0 + lr;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int c0 = 32 * s + 8 * lg;
      float x[8], y[8];
      if (row < N) {
        load8(K + row * p.sk[2] + c0 * p.sk[3], p.sk[3], vec_k, x);
        float cs[8];
        rope_load4(tab, row + shift, D2, c0 / 2, cs);
        rope_rotate8(x, cs);
        load8(V + row * p.sv[2] + c0 * p.sv[3], p.sv[3], vec_v, y);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = y[e] = 0.f;
      }
      kf[u][s] = C::make(x);
      vf[u][s] = C::make(y);
    }
  }

  // ---- K-hat^T of the whole plane (zero beyond N); zero dS columns no subtile owns ----
  const int nkv32 = round_up32(N);
#pragma unroll
  for (int it = 0; it < KITER; ++it) {
    const int u = tid + it * NT;
    const int rp = u / CPR, cc = u - rp * CPR;
    if (u < KUNITS && 2 * rp < nkv32) {
      float x0[8], x1[8], cs0[8], cs1[8];
      const int r0 = 2 * rp, r1 = 2 * rp + 1;
      if (r0 < N) {
        load8(K + r0 * p.sk[2] + 8 * cc * p.sk[3], p.sk[3], vec_k, x0);
        rope_load4(tab, r0 + shift, D2, 4 * cc, cs0);
        rope_rotate8(x0, cs0);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x0[e] = 0.f;
      }
      if (r1 < N) {
        load8(K + r1 * p.sk[2] + 8 * cc * p.sk[3], p.sk[3], vec_k, x1);
        rope_load4(tab, r1 + shift, D2, 4 * cc, cs1);
        rope_rotate8(x1, cs1);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x1[e] = 0.f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) put2b<CT>(&sKt[(8 * cc + e) * LDKT + r0], x0[e], x1[e]);
    }
  }
  {
    const int own_end = ((N + 15) / 16) * 16;   // columns [own_end, nkv32) belong to no active subtile
    const int width = nkv32 - own_end;
    for (int i = tid; i < QS * width; i += NT) {
      const int r = i / width, cidx = own_end + (i - r * width);
      C::put1(&sdS[r * LDKT + cidx], 0.f);
    }
  }

  f32x4 dvacc[KT][DT], dkacc[KT][DT];
#pragma unroll
  for (int u = 0; u < KT; ++u)
#pragma unroll
    for (int d = 0; d < DT; ++d) dvacc[u][d] = dkacc[u][d] = f32x4{0.f, 0.f, 0.f, 0.f};

  // S, dP, P, dS, dV, dK for the first NUA owned key subtiles over one query stage.
  auto sweep = [&](auto nuc, int rows) {
    constexpr int NUA = decltype(nuc)::value;
    for (int j = 0; j < rows / 32; ++j) {
      // P and dS of queries 32j + 8lg + (0..7) for each owned key, built one
      // 16-query half (h) at a time to keep the live logits small.
      Frag pf[NUA], dsf[NUA];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        f32x4 sacc[NUA], pacc[NUA];
#pragma unroll
        for (int u = 0; u < NUA; ++u) sacc[u] = pacc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int pr = 32 * j + 16 * h + lr;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const Frag a = C::lds(&sQ[pr * LDQ + 32 * s + 8 * lg]);
          const Frag b = C::lds(&sG[pr * LDQ + 32 * s + 8 * lg]);
#pragma unroll
          for (int u = 0; u < NUA; ++u) {
            sacc[u] = C::mma(a, kf[u][s], sacc[u]);
            pacc[u] = C::mma(b, vf[u][s], pacc[u]);
          }
        }
        const f32x4 l2 = *reinterpret_cast<const f32x4*>(&sL2[32 * j + 8 * lg + 4 * h]);
        const f32x4 dl = *reinterpret_cast<const f32x4*>(&sDl[32 * j + 8 * lg + 4 * h]);
#pragma unroll
        for (int u = 0; u < NUA; ++u) {
          const int kv0 = (u * NW + wave) * 16;
          const int kv = kv0 + lr;
          float pv[4], dsv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) pv[i] = fast_exp2(__builtin_fmaf(sacc[u][i], c2, -l2[i]));
          if (kv0 + 16 > N) {   // wave-uniform: only the subtile holding key N-1 masks
#pragma unroll
            for (int i = 0; i < 4; ++i) pv[i] = kv < N ? pv[i] : 0.f;
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) dsv[i] = pv[i] * (pacc[u][i] - dl[i]);
          C::set2(pf[u], 2 * h, pv[0], pv[1]);
          C::set2(pf[u], 2 * h + 1, pv[2], pv[3]);
          C::set2(dsf[u], 2 * h, dsv[0], dsv[1]);
          C::set2(dsf[u], 2 * h + 1, dsv[2], dsv[3]);
#pragma unroll
          for (int i = 0; i < 4; ++i)
            C::put_elem(&sdS[(32 * j + 8 * lg + 4 * h + i) * LDKT + kv], dsf[u], 4 * h + i);
        }
      }
      // dV^T += dO^T P ; dK-hat^T += Q-hat^T dS
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const Frag ag = C::lds(&sGt[(16 * d + lr) * LDT + 32 * j + 8 * lg]);
        const Frag aq = C::lds(&sQt[(16 * d + lr) * LDT + 32 * j + 8 * lg]);
#pragma unroll
        for (int u = 0; u < NUA; ++u) {
          dvacc[u][d] = C::mma(ag, pf[u], dvacc[u][d]);
          dkacc[u][d] = C::mma(aq, dsf[u], dkacc[u][d]);
        }
      }
    }
  };

  const int nstages = (N + QS - 1) / QS;
  for (int st = 0; st < nstages; ++st) {
    const int qb = st * QS;
    const int rows = min(QS, round_up32(N - qb));
    commit();
    if (st + 1 < nstages) prefetch(qb + QS);
    __syncthreads();

    if (nu == KT) {
      sweep(std::integral_constant<int, KT>{}, rows);
    } else if (nu == 1) {
      sweep(std::integral_constant<int, 1>{}, rows);
    }
    __syncthreads();

    // ---- dQ-hat^T[d, q] = sum_kv K-hat^T[d, kv] dS^T[kv, q] for this stage ----
    {
      constexpr int QSUB = QS / 16;                  // query subtiles per stage
      constexpr int QPW = (QSUB * DT) / NW;          // subtiles per wave (same d-subtile)
      static_assert((QSUB * DT) % NW == 0 && QSUB % QPW == 0 && QPW <= 2, "dQ job split");
      const int d = wave % DT;
      const int qs0 = (wave / DT) * QPW;
      f32x4 acc[QPW];
#pragma unroll
      for (int i = 0; i < QPW; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      int nq = 0;   // this wave's query subtiles inside the stage: a prefix (wave-uniform)
#pragma unroll
      for (int i = 0; i < QPW; ++i) nq += 16 * (qs0 + i) < rows;
      auto dq_sweep = [&](auto nqc) {
        constexpr int NQA = decltype(nqc)::value;
        for (int jj = 0; jj < nkv32 / 32; ++jj) {
          const Frag a = C::lds(&sKt[(16 * d + lr) * LDKT + 32 * jj + 8 * lg]);
#pragma unroll
          for (int i = 0; i < NQA; ++i) {
            const Frag b = C::lds(&sdS[(16 * (qs0 + i) + lr) * LDKT + 32 * jj + 8 * lg]);
            acc[i] = C::mma(a, b, acc[i]);
          }
        }
      };
      if (nq == QPW) {
        dq_sweep(std::integral_constant<int, QPW>{});
      } else if (nq > 0) {
        dq_sweep(std::integral_constant<int, 1>{});
      }
#pragma unroll
      for (int i = 0; i < QPW; ++i) {
        const int row = qb + 16 * (qs0 + i) + lr;
        if (i < nq && row < N) {
          float g4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) g4[r] = acc[i][r] * p.scale;
          rope_unrotate4(g4, tab, row + shift, D2, 8 * d + 2 * lg);
          store4(dQ + row * p.sdq[2] + (16 * d + 4 * lg) * p.sdq[3], p.sdq[3], vec_dq, g4);
        }
      }
    }
  }

  // ---- epilogue: lane holds dV / dK-hat of key kv0 + lr, channels 16d + 4lg + (0..3) ----
#pragma unroll
  for (int u = 0; u < KT; ++u) {
    const int row = (u * NW + wave) * 16 + lr;
    if (u < nu && row < N) {
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        float v4[4], g4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) { v4[r] = dvacc[u][d][r]; g4[r] = dkacc[u][d][r] * p.scale; }
        store4(dV + row * p.sdv[2] + (16 * d + 4 * lg) * p.sdv[3], p.sdv[3], vec_dv, v4);
        rope_unrotate4(g4, tab, row + shift, D2, 8 * d + 2 * lg);
        store4(dK + row * p.sdk[2] + (16 * d + 4 * lg) * p.sdk[3], p.sdk[3], vec_dk, g4);
      }
    }
  }
}

// 8 waves x 2 key subtiles = 256 keys per workgroup, 64-query stages.
constexpr int kFusedNW = 8, kFusedKT = 2, kFusedQS = 64;

int bwd_fused_rows() { return kFusedNW * kFusedKT * 16; }

template <typename IO, int CT>
static hipError_t fused_launch(const BwdParams& p, hipStream_t st) {
  const bool vec = p.vec_q && p.vec_k && p.vec_v && p.vec_o && p.vec_do && p.vec_dq && p.vec_dk &&
                   p.vec_dv;
  auto kern = vec ? bwd_fused_kernel<IO, CT, 64, kFusedNW, kFusedKT, kFusedQS, true>
                  : bwd_fused_kernel<IO, CT, 64, kFusedNW, kFusedKT, kFusedQS, false>;
  hipLaunchKernelGGL(kern, dim3(p.B * p.H), dim3(kFusedNW * 64), 0, st, p);
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
