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
// stages of 64 rows, double-buffered in LDS, one barrier per stage:
//   commit   staged registers -> LDS: Q-hat and dO rows (row-major),
//            LSE*log2(e), delta = rowsum(dO*O)
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
constexpr int kPlaneQS = 64;                  // query rows per stage
constexpr int kPlaneMaxN = kPlaneNW * 32;     // keys per workgroup
constexpr int kPlaneLD = 64 + 8;              // pitch of every LDS tile (elements)
}  // namespace

// VEC: every tensor of the call allows 16-byte vector access (decided on the
// host); the generic instantiation gathers element by element instead.
template <typename IO, int CT, bool VEC>
__global__ void __launch_bounds__(kPlaneNW * 64)
bwd_plane_kernel(const BwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  constexpr int D = 64, D2 = 32, LD = kPlaneLD, QS = kPlaneQS;
  static_assert(sizeof(S) == 2, "the plane kernel stores 16-bit operands");

  __shared__ __attribute__((aligned(16))) S sQ[2][QS * LD];          // Q-hat rows of a stage
  __shared__ __attribute__((aligned(16))) S sG[2][QS * LD];          // dO rows of a stage
  __shared__ __attribute__((aligned(16))) S sdS[2][kPlaneMaxN * LD]; // dS^T [key][query]
  __shared__ __attribute__((aligned(16))) S sK[kPlaneMaxN * LD];     // K-hat rows of the plane
  __shared__ __attribute__((aligned(16))) float sL2[2][QS];
  __shared__ __attribute__((aligned(16))) float sDl[2][QS];

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
  const float* __restrict__ lse = p.lse + (int64_t)plane * N;
  const int shift = 1 - p.has_cls;
  const float c2 = p.scale_log2;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  const int nkv32 = round_up32(N);
  const int nkb = nkv32 >> 5;                                  // 32-key blocks
  const int nstages = (N + QS - 1) / QS;
  const int kw = 32 * wave;                                    // first key of this wave
  const int nu = (kw < N) + (kw + 16 < N);                     // active 16-key subtiles

  // ---- stage staging: thread t carries row t/8, channels 8*(t%8) .. +7 of Q, dO, O ----
  const int sr = tid >> 3, sc = tid & 7;
  const IO* q_st = Q + sr * p.sq[2] + 8 * sc * p.sq[3];
  const IO* g_st = G + sr * p.sdo[2] + 8 * sc * p.sdo[3];
  const IO* o_st = O + sr * p.so[2] + 8 * sc * p.so[3];
  Raw8<IO> pq, pg, po;
  float pcs[8];
  float plse = 0.f;
  auto prefetch = [&](int qb) {
    const int gr = qb + sr;
    if (gr < N) {
      pq = load_raw8(q_st + qb * p.sq[2], p.sq[3], vec_q);
      pg = load_raw8(g_st + qb * p.sdo[2], p.sdo[3], vec_do);
      po = load_raw8(o_st + qb * p.so[2], p.so[3], vec_o);
      rope_load4(tab, gr + shift, D2, 4 * sc, pcs);
    } else {
      pq = pg = po = zero_raw8<IO>();
#pragma unroll
      for (int e = 0; e < 8; ++e) pcs[e] = 0.f;
    }
    if (tid < QS) plse = qb + tid < N ? lse[qb + tid] * kLog2e : INFINITY;
  };
  auto commit = [&](int buf) {
    float x[8], g[8], o[8];
    unpack8(pq, x);
    unpack8(pg, g);
    unpack8(po, o);
    rope_rotate8(x, pcs);
    C::put8(&sQ[buf][sr * LD + 8 * sc], x);
    C::put8(&sG[buf][sr * LD + 8 * sc], g);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d += g[e] * o[e];
    // the 8 chunks of a row are 8 consecutive lanes
    d += __shfl_xor(d, 1);
    d += __shfl_xor(d, 2);
    d += __shfl_xor(d, 4);
    if (sc == 0) sDl[buf][sr] = d;
    if (tid < QS) sL2[buf][tid] = plse;
  };

  prefetch(0);

  // ---- own keys: K-hat and V rows as B-operands; K-hat rows also go to sK
  //      (row-major, all 256 rows, zero beyond N) ----
  Frag kf[2][2], vf[2][2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = kw + 16 * u + lr;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
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
      *reinterpret_cast<decltype(kf[u][s].v)*>(&sK[row * LD + c0]) = kf[u][s].v;
    }
  }
  commit(0);

  f32x4 dvacc[2][4], dkacc[2][4];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int d = 0; d < 4; ++d) dvacc[u][d] = dkacc[u][d] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int dd = wave & 3;   // head-dim slice 16dd .. 16dd+15 of this wave's dQ tiles

  // ---- dQ of one finished stage from its dS^T tile ----
  auto dq_stage = [&](int sp) {
    const int buf = sp & 1;
    const int qb = sp * QS;
    const int rows = min(QS, round_up32(N - qb));
    const int qt0 = 2 * (wave >> 2);                  // this wave's two 16-query subtiles
    const int nq = (16 * qt0 < rows) + (16 * qt0 + 16 < rows);
    auto sweep = [&](auto nqc) {
      constexpr int NQ = decltype(nqc)::value;
      f32x4 acc[NQ];
#pragma unroll
      for (int i = 0; i < NQ; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < kPlaneMaxN / 32; ++kb) {
        if (kb < nkb) {
          // A = K-hat^T rows 16dd.., k = keys 32kb + 8lg + (0..7)
          const Frag a = C::tr(&sK[tr_offset(32 * kb + 8 * lg, 16 * dd, LD, lr)],
                               &sK[tr_offset(32 * kb + 8 * lg + 4, 16 * dd, LD, lr)]);
#pragma unroll
          for (int i = 0; i < NQ; ++i) {
            const S* t = &sdS[buf][0];
            const int c0 = 16 * (qt0 + i);
            const Frag b = C::tr(t + tr_offset(32 * kb + 8 * lg, c0, LD, lr),
                                 t + tr_offset(32 * kb + 8 * lg + 4, c0, LD, lr));
            acc[i] = C::mma(a, b, acc[i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int row = qb + 16 * (qt0 + i) + lr;
        if (row < N) {
          float g4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) g4[r] = acc[i][r] * p.scale;
          rope_unrotate4(g4, tab, row + shift, D2, 8 * dd + 2 * lg);
          store4(dQ + row * p.sdq[2] + (16 * dd + 4 * lg) * p.sdq[3], p.sdq[3], vec_dq, g4);
        }
      }
    };
    if (nq == 2) {
      sweep(std::integral_constant<int, 2>{});
    } else if (nq == 1) {
      sweep(std::integral_constant<int, 1>{});
    }
  };

  // ---- S, dP, P, dS, dV, dK for the wave's first NUA subtiles over one stage ----
  auto sweep_keys = [&](auto nuc, int buf, int rows) {
    constexpr int NUA = decltype(nuc)::value;
    const S* q = &sQ[buf][0];
    const S* g = &sG[buf][0];
    S* ds = &sdS[buf][0];
    if constexpr (NUA > 0) {
#pragma unroll
    for (int j = 0; j < QS / 32; ++j) {
      if (32 * j < rows) {
        Frag pf[NUA], dsf[NUA];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          f32x4 sacc[NUA], pacc[NUA];
#pragma unroll
          for (int u = 0; u < NUA; ++u) sacc[u] = pacc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
          const int qr = 32 * j + 16 * h + lr;
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const Frag a = C::lds(q + qr * LD + 32 * s + 8 * lg);
            const Frag b = C::lds(g + qr * LD + 32 * s + 8 * lg);
#pragma unroll
            for (int u = 0; u < NUA; ++u) {
              sacc[u] = C::mma(a, kf[u][s], sacc[u]);
              pacc[u] = C::mma(b, vf[u][s], pacc[u]);
            }
          }
          const int q0 = 32 * j + 16 * h + 4 * lg;   // queries q0 .. q0+3 in this lane
          const f32x4 l2 = *reinterpret_cast<const f32x4*>(&sL2[buf][q0]);
          const f32x4 dl = *reinterpret_cast<const f32x4*>(&sDl[buf][q0]);
#pragma unroll
          for (int u = 0; u < NUA; ++u) {
            const int kv0 = kw + 16 * u;
            float pv[4], dsv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) pv[i] = fast_exp2(__builtin_fmaf(sacc[u][i], c2, -l2[i]));
            if (kv0 + 16 > N) {   // wave-uniform: only the subtile holding key N-1 masks
#pragma unroll
              for (int i = 0; i < 4; ++i) pv[i] = kv0 + lr < N ? pv[i] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) dsv[i] = pv[i] * (pacc[u][i] - dl[i]);
            C::set2(pf[u], 2 * h, pv[0], pv[1]);
            C::set2(pf[u], 2 * h + 1, pv[2], pv[3]);
            C::set2(dsf[u], 2 * h, dsv[0], dsv[1]);
            C::set2(dsf[u], 2 * h + 1, dsv[2], dsv[3]);
            C::put4(ds + (kv0 + lr) * LD + q0, dsf[u], h);
          }
        }
        // dV^T += dO^T P ; dK-hat^T += Q-hat^T dS  (k = queries 32j + 16h + 4lg + e)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const int o0 = tr_offset(32 * j + 4 * lg, 16 * d, LD, lr);
          const int o1 = tr_offset(32 * j + 16 + 4 * lg, 16 * d, LD, lr);
          const Frag ag = C::tr(g + o0, g + o1);
          const Frag aq = C::tr(q + o0, q + o1);
#pragma unroll
          for (int u = 0; u < NUA; ++u) {
            dvacc[u][d] = C::mma(ag, pf[u], dvacc[u][d]);
            dkacc[u][d] = C::mma(aq, dsf[u], dkacc[u][d]);
          }
        }
      }
    }
    }
    // subtiles without keys < N still cover columns < nkv32 of dS^T: zero them
#pragma unroll
    for (int u = NUA; u < 2; ++u) {
      const int kv0 = kw + 16 * u;
      if (kv0 < nkv32) {
        const Frag z = C::zero();
#pragma unroll
        for (int j = 0; j < QS / 32; ++j)
          if (32 * j < rows) {
            C::put4(ds + (kv0 + lr) * LD + 32 * j + 4 * lg, z, 0);
            C::put4(ds + (kv0 + lr) * LD + 32 * j + 16 + 4 * lg, z, 0);
          }
      }
    }
  };

  for (int st = 0; st < nstages; ++st) {
    const int buf = st & 1;
    const int qb = st * QS;
    if (st > 0) commit(buf);
    __syncthreads();
    if (st + 1 < nstages) prefetch(qb + QS);
    if (st > 0) dq_stage(st - 1);
    const int rows = min(QS, round_up32(N - qb));
    if (nu == 2) {
      sweep_keys(std::integral_constant<int, 2>{}, buf, rows);
    } else if (nu == 1) {
      sweep_keys(std::integral_constant<int, 1>{}, buf, rows);
    } else {
      sweep_keys(std::integral_constant<int, 0>{}, buf, rows);
    }
  }
  __syncthreads();
  dq_stage(nstages - 1);

  // ---- epilogue: lane holds dV / dK-hat of key kv0 + lr, channels 16d + 4lg + (0..3) ----
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int row = kw + 16 * u + lr;
    if (u < nu && row < N) {
#pragma unroll
      for (int d = 0; d < 4; ++d) {
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

int bwd_fused_rows() { return kPlaneMaxN; }

template <typename IO, int CT>
static hipError_t fused_launch(const BwdParams& p, hipStream_t st) {
  const bool vec = p.vec_q && p.vec_k && p.vec_v && p.vec_o && p.vec_do && p.vec_dq && p.vec_dk &&
                   p.vec_dv;
  auto kern = vec ? bwd_plane_kernel<IO, CT, true> : bwd_plane_kernel<IO, CT, false>;
  hipLaunchKernelGGL(kern, dim3(p.B * p.H), dim3(kPlaneNW * 64), 0, st, p);
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
