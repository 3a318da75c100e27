// Forward kernel: O = softmax(scale * (R Q)(R K)^T) V and LSE, fused 2D RoPE.
//
// Reference behaviour followed: _attn_fwd in "fa_rope_full .py" (FA:91-315):
// Q/K pair rotation with the CLS row bypassing RoPE (FA:176-202, FA:248-272),
// scaled logits with padded key columns masked out (FA:275-277), online
// softmax with a running max (FA:280-305) and the per-row log-sum-exp stored
// for the backward pass (FA:308-309).
//
// gfx950 design:
//  * A workgroup (NW waves) sweeps NW*QT q-subtiles of 16 rows of one (b, h)
//    plane per pass; wave w takes subtiles w, w+NW, ... of the pass, so the
//    ragged tail (N = 1 + H_img^2) is spread over the waves.  Rotated Q rows
//    stay in registers as MFMA B-operands during a pass.  For N <= 256 one
//    workgroup owns the whole plane and makes ceil(N/16 / (NW*QT)) passes
//    over the K-hat/V^T it keeps in LDS, so K and V are staged once.
//  * K and V are consumed in chunks of KC rows through a ring of NBUF LDS
//    slots.  Chunk c+1 is loaded from HBM into registers while chunk c is
//    being computed (one barrier per chunk); for N <= 256 the ring holds
//    the whole plane.  K is rotated once per workgroup on its way into LDS
//    (row-major K-hat, rows permuted so that the 16 rows one MFMA reads are
//    consecutive: no bank conflicts); V is stored transposed (V^T), two keys
//    per 32-bit LDS write.
//  * Logits are computed transposed, S^T = K-hat Q-hat^T, with key
//    kv = 8*(r/4) + 4*h + r%4 of a 32-key block in A-row r of half h.  Lane
//    group lg then holds keys 8*lg .. 8*lg+7 of its query column: exactly the
//    B-operand of O^T += V^T P^T, so P never leaves registers and each V^T
//    fragment is one 16-byte LDS read shared by all QT subtiles.
//  * One query row per lane: the row max needs two cross-lane steps per
//    32-key block.  Softmax runs in base 2 (log2(e) folded into the scale)
//    with fp32 state and accumulator; O and the row sum are rescaled only
//    when the running max grows by more than 2^8 (P <= 256 otherwise), so
//    the rescale is rare after the first block.
#include <type_traits>

#include "common.h"
#include "params.h"

namespace farope {

template <int CT> __device__ __forceinline__ void put2(typename Comp<CT>::S* p, float a, float b);
template <> __device__ __forceinline__ void put2<DT_BF16>(bf16* p, float a, float b) {
  typedef bf16 bf16x2 __attribute__((ext_vector_type(2)));
  bf16x2 v;
  v[0] = (bf16)a;
  v[1] = (bf16)b;
  *reinterpret_cast<bf16x2*>(p) = v;
}
template <> __device__ __forceinline__ void put2<DT_F16>(f16* p, float a, float b) {
  typedef f16 f16x2 __attribute__((ext_vector_type(2)));
  f16x2 v;
  v[0] = (f16)a;
  v[1] = (f16)b;
  *reinterpret_cast<f16x2*>(p) = v;
}
template <> __device__ __forceinline__ void put2<DT_F32>(float* p, float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  f32x2 v;
  v[0] = a;
  v[1] = b;
  *reinterpret_cast<f32x2*>(p) = v;
}

// Physical LDS row of key r of a chunk: within each 32-key block,
// r = 8a + 4h + i is stored at 16h + 4a + i.
__device__ __forceinline__ int kperm(int r) {
  return (r & ~31) | ((r & 4) << 2) | ((r & 24) >> 1) | (r & 3);
}

constexpr float kRescaleSlack = 8.0f;   // log2 units: P <= 2^8 between rescales

template <typename IO, int CT, int D, int NW, int QT, int KC, int NBUF>
__global__ void __launch_bounds__(NW * 64, 2)
fwd_kernel(const FwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  constexpr int KS = D / 32;          // k-steps of 32 channels
  constexpr int DT = D / 16;          // 16-channel output subtiles
  constexpr int D2 = D / 2;
  constexpr int PADE = 16 / sizeof(S);
  constexpr int LDK = D + PADE;       // K-hat row pitch (elements)
  constexpr int LDV = KC + PADE;      // V^T row pitch
  constexpr int NT = NW * 64;
  constexpr int CPR = D / 8;          // 8-channel chunks per row
  constexpr int UNITS = (KC / 2) * CPR;   // (row pair, chunk) staging units per KV chunk
  constexpr int ITER = (UNITS + NT - 1) / NT;
  constexpr bool kPlane = NBUF * KC >= 256;   // LDS ring holds a whole plane (host: N <= 256)
  static_assert(KC % 32 == 0, "KV chunk must be a multiple of 32 keys");

  __shared__ __attribute__((aligned(16))) S sK[NBUF][KC * LDK];
  __shared__ __attribute__((aligned(16))) S sVt[NBUF][D * LDV];

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
  const bool vec_k = p.vec_k, vec_v = p.vec_v;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;

  // ---- KV chunk prefetch registers: two rows x 8 channels of K, V, (cos, sin) ----
  Raw8<IO> pk[ITER][2], pv[ITER][2];
  float pcs[ITER][2][8];
  auto prefetch = [&](int kvb) {
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int u = tid + it * NT;
      const int rp = u / CPR, cc = u - rp * CPR;
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        const int gr = kvb + 2 * rp + x;
        if (u < UNITS && gr < N) {
          pk[it][x] = load_raw8(K + gr * p.sk[2] + 8 * cc * p.sk[3], p.sk[3], vec_k);
          pv[it][x] = load_raw8(V + gr * p.sv[2] + 8 * cc * p.sv[3], p.sv[3], vec_v);
          rope_load4(tab, gr + shift, D2, 4 * cc, pcs[it][x]);
        } else {
          pk[it][x] = zero_raw8<IO>();
          pv[it][x] = zero_raw8<IO>();
#pragma unroll
          for (int e = 0; e < 8; ++e) pcs[it][x][e] = 0.f;
        }
      }
    }
  };
  auto commit = [&](int slot) {
#pragma unroll
    for (int it = 0; it < ITER; ++it) {
      const int u = tid + it * NT;
      const int rp = u / CPR, cc = u - rp * CPR;
      if (u < UNITS) {
        float xv[2][8];
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          float xk[8];
          unpack8(pk[it][x], xk);
          rope_rotate8(xk, pcs[it][x]);
          C::put8(&sK[slot][kperm(2 * rp + x) * LDK + 8 * cc], xk);
          unpack8(pv[it][x], xv[x]);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) put2<CT>(&sVt[slot][(8 * cc + e) * LDV + 2 * rp], xv[0][e], xv[1][e]);
      }
    }
  };

  Frag qf[QT][KS];
  float m_run[QT], l_run[QT];
  f32x4 oacc[QT][DT];
  const float c2 = p.scale_log2;
  const int nsub = (N + 15) / 16;            // 16-row q-subtiles of the plane
  // Pass `ps` of this workgroup covers subtiles base + t*NW + wave, t < QT.
  auto pass_base = [&](int ps) { return (qblk + ps) * NW * QT; };

  // ---- rotated Q rows of one pass -> B-operand fragments; returns the number
  //      of active subtiles of this wave (a prefix t < nt, wave-uniform) ----
  auto load_q = [&](int ps) {
    int nt = 0;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int sub = pass_base(ps) + t * NW + wave;
      nt += sub < nsub;
      const int row = sub * 16 + lr;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float x[8];
        const int c0 = 32 * s + 8 * lg;
        if (row < N) {
          load8(Q + row * p.sq[2] + c0 * p.sq[3], p.sq[3], p.vec_q, x);
          float cs[8];
          rope_load4(tab, row + shift, D2, c0 / 2, cs);
          rope_rotate8(x, cs);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] = 0.f;
        }
        qf[t][s] = C::make(x);
      }
      m_run[t] = -INFINITY;
      l_run[t] = 0.f;
#pragma unroll
      for (int d = 0; d < DT; ++d) oacc[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    return nt;
  };

  // One KV chunk for the first NTA subtiles (NTA is a compile-time count so
  // the MFMA / softmax stream carries no per-subtile guards).
  auto chunk = [&](auto ntc, const S* __restrict__ cK, const S* __restrict__ cV, int kvb) {
    constexpr int NTA = decltype(ntc)::value;
    const int nblk = min(KC, round_up32(N - kvb)) / 32;
    for (int j = 0; j < nblk; ++j) {
      // ---- S^T = K-hat Q-hat^T for 32 keys (each K-hat fragment feeds NTA MFMAs) ----
      f32x4 sacc[NTA][2];
#pragma unroll
      for (int t = 0; t < NTA; ++t) sacc[t][0] = sacc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const Frag a = C::lds(&cK[(32 * j + 16 * h + lr) * LDK + 32 * s + 8 * lg]);
#pragma unroll
          for (int t = 0; t < NTA; ++t) sacc[t][h] = C::mma(a, qf[t][s], sacc[t][h]);
        }
      }
      // ---- online softmax; lane holds keys kvb + 32j + 8lg + (0..7) of its row ----
      const int kbase = kvb + 32 * j + 8 * lg;
      const bool masked = kvb + 32 * j + 32 > N;
      Frag pf[NTA];
#pragma unroll
      for (int t = 0; t < NTA; ++t) {
        float sv[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[4 * h + i] = sacc[t][h][i];
        if (masked) {
#pragma unroll
          for (int e = 0; e < 8; ++e) sv[e] = kbase + e < N ? sv[e] : -INFINITY;
        }
        float mx = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                         fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
        mx = group4_max(mx) * c2;
        if (__any(mx > m_run[t] + kRescaleSlack)) {
          const float mnew = fmaxf(m_run[t], mx);
          const float alpha = fast_exp2(m_run[t] - mnew);
          l_run[t] *= alpha;
#pragma unroll
          for (int d = 0; d < DT; ++d) oacc[t][d] *= alpha;
          m_run[t] = mnew;
        }
        float pv8[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv8[e] = fast_exp2(__builtin_fmaf(sv[e], c2, -m_run[t]));
          l_run[t] += pv8[e];
        }
        pf[t] = C::make(pv8);
      }
      // ---- O^T += V^T P^T (each V^T fragment feeds NTA MFMAs) ----
#pragma unroll
      for (int d = 0; d < DT; ++d) {
        const Frag a = C::lds(&cV[(16 * d + lr) * LDV + 32 * j + 8 * lg]);
#pragma unroll
        for (int t = 0; t < NTA; ++t) oacc[t][d] = C::mma(a, pf[t], oacc[t][d]);
      }
    }
  };
  auto run_chunk = [&](int nt, int slot, int kvb) {
    if (nt == QT) {
      chunk(std::integral_constant<int, QT>{}, sK[slot], sVt[slot], kvb);
    } else if (nt > 0) {
      if constexpr (QT >= 3) {
        if (nt == 2) { chunk(std::integral_constant<int, 2>{}, sK[slot], sVt[slot], kvb); return; }
      }
      chunk(std::integral_constant<int, 1>{}, sK[slot], sVt[slot], kvb);
    }
  };

  // ---- epilogue of a pass: lane holds O[row][16d + 4lg + (0..3)] ----
  auto store_pass = [&](int ps, int nt) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const float l = group4_sum(l_run[t]);
      const int row = (pass_base(ps) + t * NW + wave) * 16 + lr;
      if (t < nt && row < N) {
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
  };

  prefetch(0);
  int nt = load_q(0);

  // ---- pass 0: software-pipelined over KV chunks ----
  const int nchunks = (N + KC - 1) / KC;
  for (int c = 0; c < nchunks; ++c) {
    const int slot = c % NBUF;
    const int kvb = c * KC;
    commit(slot);
    if (c + 1 < nchunks) prefetch(kvb + KC);
    __syncthreads();
    run_chunk(nt, slot, kvb);
  }
  store_pass(0, nt);

  // ---- further passes (plane-resident variant: every chunk is still in LDS) ----
  if constexpr (kPlane) {
    const int npass = (nsub - pass_base(0) + NW * QT - 1) / (NW * QT);
    for (int ps = 1; ps < npass; ++ps) {
      nt = load_q(ps);
      for (int c = 0; c < nchunks; ++c) run_chunk(nt, c, c * KC);
      store_pass(ps, nt);
    }
  }
}

// ---------------------------------------------------------------------------
// Tile table for the forward pass: (NW, QT, KC, NBUF) per head_dim/variant.
// ---------------------------------------------------------------------------
template <int D, int VAR> struct FwdShape;
// plane-resident: 4 slots x 64 keys = 256 keys in LDS; 4 waves x 2 subtiles
// = 128 query rows per pass, ceil(N/128) passes over the resident K-hat/V^T.
template <> struct FwdShape<64, FWD_PLANE> { static constexpr int NW = 4, QT = 2, KC = 64, NBUF = 4; };
template <> struct FwdShape<64, FWD_STREAM> { static constexpr int NW = 4, QT = 2, KC = 64, NBUF = 2; };
template <> struct FwdShape<128, FWD_STREAM> { static constexpr int NW = 4, QT = 1, KC = 32, NBUF = 2; };

int fwd_block_rows(int D, int variant) {
  if (D == 64 && variant == FWD_PLANE) {
    using SH = FwdShape<64, FWD_PLANE>;
    return SH::NBUF * SH::KC;   // one workgroup per plane
  }
  if (D == 64) {
    using SH = FwdShape<64, FWD_STREAM>;
    return SH::NW * SH::QT * 16;
  }
  using SH = FwdShape<128, FWD_STREAM>;
  return SH::NW * SH::QT * 16;
}

template <typename IO, int CT, int D, int VAR>
static hipError_t fwd_launch(const FwdParams& p, hipStream_t st) {
  using SH = FwdShape<D, VAR>;
  const int grid = p.B * p.H * p.n_blk;
  hipLaunchKernelGGL((fwd_kernel<IO, CT, D, SH::NW, SH::QT, SH::KC, SH::NBUF>), dim3(grid),
                     dim3(SH::NW * 64), 0, st, p);
  return hipGetLastError();
}

template <typename IO, int CT>
static hipError_t fwd_shape(const FwdParams& p, int D, int variant, hipStream_t st) {
  if (D == 64)
    return variant == FWD_PLANE ? fwd_launch<IO, CT, 64, FWD_PLANE>(p, st)
                                : fwd_launch<IO, CT, 64, FWD_STREAM>(p, st);
  return fwd_launch<IO, CT, 128, FWD_STREAM>(p, st);
}

template <typename IO>
static hipError_t fwd_ct(const FwdParams& p, int ct, int D, int variant, hipStream_t st) {
  switch (ct) {
    case DT_BF16: return fwd_shape<IO, DT_BF16>(p, D, variant, st);
    case DT_F16: return fwd_shape<IO, DT_F16>(p, D, variant, st);
    default: return fwd_shape<IO, DT_F32>(p, D, variant, st);
  }
}

hipError_t launch_fwd(const FwdParams& p, int io, int ct, int D, int variant, hipStream_t st) {
  switch (io) {
    case DT_BF16: return fwd_ct<bf16>(p, ct, D, variant, st);
    case DT_F16: return fwd_ct<f16>(p, ct, D, variant, st);
    default: return fwd_ct<float>(p, ct, D, variant, st);
  }
}

}  // namespace farope
