// Forward kernel: O = softmax(scale * (R Q)(R K)^T) V and LSE, fused 2D RoPE.
//
// Reference behaviour followed: _attn_fwd in "fa_rope_full .py" (FA:91-315):
// Q/K pair rotation with the CLS row bypassing RoPE (FA:176-202, FA:248-272),
// scaled logits with padded key columns masked out (FA:275-277), online
// softmax with a running max (FA:280-305) and the per-row log-sum-exp stored
// for the backward pass (FA:308-309).
//
// gfx950 design:
//  * Each wave owns QT q-subtiles of 16 rows.  Its rotated Q rows live in
//    registers as MFMA B-operands for the whole kernel.
//  * K is rotated once per workgroup while it is staged into LDS (row-major
//    K-hat), V is staged transposed (V^T), both in compute precision.
//  * Logits are computed transposed, S^T = K-hat Q-hat^T, with the K-hat rows
//    of each 32-key block fed in the order kv = 8*(r/4) + 4*h + r%4.  That
//    leaves lane group lg holding keys 8*lg .. 8*lg+7 of its query column,
//    which is exactly the B-operand layout of O^T += V^T P^T: P never
//    leaves registers and V^T is read as 16-byte LDS vectors.
//  * Each lane owns one query row, so softmax statistics need only two
//    cross-lane steps (lanes lr, lr+16, lr+32, lr+48) per 32-key block.
//  * Softmax runs in base 2 with log2(e) folded into the scale; fp32 state,
//    fp32 O accumulator.
#include "common.h"
#include "params.h"

namespace farope {

template <typename IO, int CT, int D, int NW, int QT, int KVS>
__global__ void __launch_bounds__(NW * 64)
fwd_kernel(const FwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  constexpr int KS = D / 32;          // k-steps of 32 channels
  constexpr int DT = D / 16;          // 16-channel output subtiles
  constexpr int D2 = D / 2;
  constexpr int PADE = 16 / sizeof(S);
  constexpr int LDK = D + PADE;       // K-hat row pitch (elements)
  constexpr int LDV = KVS + PADE;     // V^T row pitch
  constexpr int NT = NW * 64;
  constexpr int CPR = D / 8;          // 8-channel chunks per row
  constexpr int ITER = (KVS * CPR + NT - 1) / NT;
  constexpr int QROWS = NW * QT * 16;

  __shared__ __attribute__((aligned(16))) S sK[KVS * LDK];
  __shared__ __attribute__((aligned(16))) S sVt[D * LDV];

  const int N = p.N;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int plane = tile / p.n_blk;
  const int qblk = tile - plane * p.n_blk;
  const int bb = plane / p.H, hh = plane - bb * p.H;
  const IO* __restrict__ Q = static_cast<const IO*>(p.q) + bb * p.sq[0] + hh * p.sq[1];
  const IO* __restrict__ K = static_cast<const IO*>(p.k) + bb * p.sk[0] + hh * p.sk[1];
  const IO* __restrict__ V = static_cast<const IO*>(p.v) + bb * p.sv[0] + hh * p.sv[1];
  IO* __restrict__ O = static_cast<IO*>(p.o) + bb * p.so[0] + hh * p.so[1];
  const float* __restrict__ tab = p.rope;
  const int shift = 1 - p.has_cls;    // table row of token s is s + shift

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // ---- rotated Q rows -> B-operand fragments (registers) ----
  Frag qf[QT][KS];
  int qrow[QT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const int q0 = qblk * QROWS + (wave * QT + t) * 16;
    qrow[t] = q0 + lr;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      float x[8];
      const int c0 = 32 * s + 8 * lg;
      if (qrow[t] < N) {
        load8(Q + qrow[t] * p.sq[2] + c0 * p.sq[3], p.sq[3], p.vec_q, x);
        float cs[8];
        rope_load4(tab, qrow[t] + shift, D2, c0 / 2, cs);
        rope_rotate8(x, cs);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      }
      qf[t][s] = C::make(x);
    }
  }
  const bool wave_active = qblk * QROWS + wave * QT * 16 < N;

  float m_run[QT], l_run[QT];
  f32x4 oacc[QT][DT];
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    m_run[t] = -INFINITY;
    l_run[t] = 0.f;
#pragma unroll
    for (int d = 0; d < DT; ++d) oacc[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  for (int kvb = 0; kvb < N; kvb += KVS) {
    const int rows = min(KVS, round_up32(N - kvb));
    if (kvb > 0) __syncthreads();   // previous stage fully consumed

    // ---- stage K-hat (row-major) and V^T into LDS; rows >= N are zero ----
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
          C::put8(&sK[r * LDK + 8 * cc], xk[it]);
#pragma unroll
          for (int e = 0; e < 8; ++e) C::put1(&sVt[(8 * cc + e) * LDV + r], xv[it][e]);
        }
      }
    }
    __syncthreads();
    if (!wave_active) continue;

    for (int j = 0; j < rows / 32; ++j) {
      // ---- S^T = K-hat Q-hat^T for 32 keys ----
      f32x4 sacc[QT][2];
#pragma unroll
      for (int t = 0; t < QT; ++t) sacc[t][0] = sacc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int kl = 32 * j + 8 * (lr >> 2) + 4 * h + (lr & 3);
          const Frag a = C::lds(&sK[kl * LDK + 32 * s + 8 * lg]);
#pragma unroll
          for (int t = 0; t < QT; ++t) sacc[t][h] = C::mma(a, qf[t][s], sacc[t][h]);
        }
      }
      // ---- online softmax; lane holds keys kvb + 32j + 8lg + (0..7) ----
      const int kbase = kvb + 32 * j + 8 * lg;
      const bool full = kvb + 32 * j + 32 <= N;
      Frag pf[QT];
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        float sv[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x = sacc[t][h][i] * p.scale_log2;
            sv[4 * h + i] = (full || kbase + 4 * h + i < N) ? x : -INFINITY;
          }
        float mx = sv[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sv[e]);
        mx = group4_max(mx);
        const float mnew = fmaxf(m_run[t], mx);
        const float alpha = fast_exp2(m_run[t] - mnew);
        float pv[8], ps = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = fast_exp2(sv[e] - mnew);
          ps += pv[e];
        }
        l_run[t] = l_run[t] * alpha + ps;
        m_run[t] = mnew;
#pragma unroll
        for (int d = 0; d < DT; ++d) oacc[t][d] *= alpha;
        pf[t] = C::make(pv);
      }
      // ---- O^T += V^T P^T ----
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const Frag a = C::lds(&sVt[(16 * d + lr) * LDV + 32 * j + 8 * lg]);
#pragma unroll
        for (int t = 0; t < QT; ++t) oacc[t][d] = C::mma(a, pf[t], oacc[t][d]);
      }
    }
  }

  // ---- epilogue: lane holds O[qrow][16d + 4lg + (0..3)] ----
#pragma unroll
  for (int t = 0; t < QT; ++t) {
    const float l = group4_sum(l_run[t]);
    const int row = qrow[t];
    if (row < N) {
      const float inv = 1.f / l;
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        float o4[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o4[r] = oacc[t][d][r] * inv;
        store4(O + row * p.so[2] + (16 * d + 4 * lg) * p.so[3], p.so[3], p.vec_o, o4);
      }
      if (lg == 0) p.lse[(int64_t)plane * N + row] = (m_run[t] + fast_log2(l)) * kLn2;
    }
  }
}

// ---------------------------------------------------------------------------
// Tile table for the forward pass.
// ---------------------------------------------------------------------------
template <int D> struct FwdShape;
//                        NW  QT  KVS
template <> struct FwdShape<64> {
  static constexpr int PLANE_NW = 8, PLANE_QT = 2, PLANE_KVS = 256;
  static constexpr int STREAM_NW = 4, STREAM_QT = 2, STREAM_KVS = 64;
};
template <> struct FwdShape<128> {
  static constexpr int PLANE_NW = 8, PLANE_QT = 1, PLANE_KVS = 128;   // unused: D=128 streams
  static constexpr int STREAM_NW = 4, STREAM_QT = 2, STREAM_KVS = 64;
};

int fwd_block_rows(int D, int variant) {
  if (D == 64)
    return variant == FWD_PLANE ? FwdShape<64>::PLANE_NW * FwdShape<64>::PLANE_QT * 16
                                : FwdShape<64>::STREAM_NW * FwdShape<64>::STREAM_QT * 16;
  return FwdShape<128>::STREAM_NW * FwdShape<128>::STREAM_QT * 16;
}

template <typename IO, int CT, int D>
static hipError_t fwd_dispatch(const FwdParams& p, int variant, hipStream_t st) {
  using SH = FwdShape<D>;
  const int grid = p.B * p.H * p.n_blk;
  if (D == 64 && variant == FWD_PLANE) {
    hipLaunchKernelGGL((fwd_kernel<IO, CT, D, SH::PLANE_NW, SH::PLANE_QT, SH::PLANE_KVS>),
                       dim3(grid), dim3(SH::PLANE_NW * 64), 0, st, p);
  } else {
    hipLaunchKernelGGL((fwd_kernel<IO, CT, D, SH::STREAM_NW, SH::STREAM_QT, SH::STREAM_KVS>),
                       dim3(grid), dim3(SH::STREAM_NW * 64), 0, st, p);
  }
  return hipGetLastError();
}

template <typename IO, int D>
static hipError_t fwd_ct(const FwdParams& p, int ct, int variant, hipStream_t st) {
  switch (ct) {
    case DT_BF16: return fwd_dispatch<IO, DT_BF16, D>(p, variant, st);
    case DT_F16: return fwd_dispatch<IO, DT_F16, D>(p, variant, st);
    default: return fwd_dispatch<IO, DT_F32, D>(p, variant, st);
  }
}

template <int D>
static hipError_t fwd_io(const FwdParams& p, int io, int ct, int variant, hipStream_t st) {
  switch (io) {
    case DT_BF16: return fwd_ct<bf16, D>(p, ct, variant, st);
    case DT_F16: return fwd_ct<f16, D>(p, ct, variant, st);
    default: return fwd_ct<float, D>(p, ct, variant, st);
  }
}

hipError_t launch_fwd(const FwdParams& p, int io, int ct, int D, int variant, hipStream_t st) {
  if (D == 64) return fwd_io<64>(p, io, ct, variant, st);
  return fwd_io<128>(p, io, ct, FWD_STREAM, st);
}

}  // namespace farope
