// Tail rows: the last N % R rows of a plane when they are few (R = rows per
// block of the forward / dQ kernels, keys per block of the dK/dV kernel).
//
// The block kernels stage all keys (or queries) of a plane through LDS for
// every block, so a block that holds one row (N = 1025 = 4 * 256 + 1, the
// 32 x 32 grid plus the CLS token) costs as much as a full one: 14% of the
// N = 1025, D = 128 step.  Here those rows are computed without staging: one
// workgroup per (plane, row), its groups of D / 8 lanes (8 channels per lane)
// walking the plane's rows straight from global memory, in fp32.  Same
// mathematics as the block kernels (reference: FA:280-305 forward, FA:623-662
// dK/dV, FA:958-993 dQ; the CLS row is not rotated, FA:176-202):
//   forward   O_r = softmax_j(q-hat_r . k-hat_j * scale) V, LSE_r
//   rows      delta_r = dO_r . O_r; dQ_r = scale R^T sum_j dS_rj k-hat_j
//   keys      dV_c = sum_i P_ic dO_i; dK_c = scale R^T sum_i dS_ic q-hat_i
// with P_ij = exp(S_ij - LSE_i), dS = P (dP - delta), dP_ij = dO_i . v_j.
// Rotated rows stay fp32 here (the block kernels round them to the compute
// type), so these rows are at least as accurate as the others.  The lane
// groups' partial results are merged in LDS in a fixed order: deterministic.
#include "common.h"
#include "params.h"

namespace farope {

namespace {

// 8 waves: two such workgroups fit on a CU, so one launch of B*H*R workgroups
// (384 for the N = 1025 bench planes) is resident at once.
constexpr int kTailThreads = 512;
// rows of the plane in flight per lane group: each trip loads kTailU rows
// (clamped to the plane, so the loads are unconditional) before using them
constexpr int kTailU = 4;

// Sum over each aligned group of W consecutive lanes (W a power of two <= 32),
// result in every lane of the group: DPP within 16-lane rows (quad
// permutations, half-row mirror, row mirror), one lane swap across rows.
template <int W>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (W >= 2) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
  if constexpr (W >= 4) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
  if constexpr (W >= 8) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
  if constexpr (W >= 16) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
  if constexpr (W >= 32) x += __shfl_xor(x, 16);
  return x;
}

template <typename IO>
__device__ __forceinline__ const IO* plane_row(const void* b, const int64_t* s, int plane, int H,
                                               int row) {
  const int bb = plane / H, hh = plane - bb * H;
  return static_cast<const IO*>(b) + bb * s[0] + hh * s[1] + (int64_t)row * s[2];
}

// channels 8c .. 8c+7 of a row as fp32.  VEC (decided on the host for every
// tensor of the call): unit channel stride and 16-byte alignment, one vector
// load; otherwise element by element.
template <bool VEC, typename IO>
__device__ __forceinline__ void load_row8(const IO* row, const int64_t* s, int c, float (&x)[8]) {
  unpack8(load_raw8(row + 8 * c * s[3], s[3], VEC), x);
}

// the same channels rotated with table row trow (token + 1 - has_cls; row 0
// is the identity that the CLS token uses)
template <bool VEC, typename IO, int D>
__device__ __forceinline__ void load_rot8(const IO* row, const int64_t* s, int c, const float* tab,
                                          int trow, float (&x)[8]) {
  load_row8<VEC>(row, s, c, x);
  float cs[8];
  rope_load4(tab, trow, D / 2, 4 * c, cs);
  rope_rotate8(x, cs);
}

// LDS scratch for merging: per lane group, D channels (two vectors for the
// dK/dV kernel) and two scalars
template <int D>
struct TailLds {
  static constexpr int G = kTailThreads / (D / 8);   // lane groups per workgroup
  float v0[G * D];
  float v1[G * D];
  float s0[G];
  float s1[G];
};

template <typename IO, int D, bool VEC>
__global__ void __launch_bounds__(kTailThreads) fwd_tail_kernel(const FwdParams p, int row0) {
  constexpr int LPR = D / 8, G = kTailThreads / LPR;
  __shared__ TailLds<D> sm;
  const int tid = thread_id(), grp = tid / LPR, c = tid % LPR;
  const int N = p.N, R = N - row0, shift = 1 - p.has_cls;
  const int plane = block_id() / R, r = row0 + block_id() % R;

  // q-hat channels of this lane, in log2 units of the logits
  float q[8];
  load_rot8<VEC, IO, D>(plane_row<IO>(p.q, p.sq, plane, p.H, r), p.sq, c, p.rope, r + shift, q);
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] *= p.scale_log2;

  float m = -INFINITY, l = 0.f, o[8] = {};
  for (int j0 = grp; j0 < N; j0 += kTailU * G) {
    float k[kTailU][8], v[kTailU][8], s[kTailU];
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      const int j = min(j0 + u * G, N - 1);
      load_rot8<VEC, IO, D>(plane_row<IO>(p.k, p.sk, plane, p.H, j), p.sk, c, p.rope, j + shift, k[u]);
      load_row8<VEC>(plane_row<IO>(p.v, p.sv, plane, p.H, j), p.sv, c, v[u]);
    }
    float mx = m;
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      float x = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) x = __builtin_fmaf(q[e], k[u][e], x);
      s[u] = j0 + u * G < N ? group_sum<LPR>(x) : -INFINITY;
      mx = fmaxf(mx, s[u]);
    }
    const float a = fast_exp2(m - mx);
    l *= a;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= a;
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      const float pj = fast_exp2(s[u] - mx);
      l += pj;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(pj, v[u][e], o[e]);
    }
    m = mx;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) sm.v0[grp * D + 8 * c + e] = o[e];
  if (c == 0) {
    sm.s0[grp] = m;
    sm.s1[grp] = l;
  }
  __syncthreads();
  // merge: M = max_g m_g, L = sum_g l_g 2^(m_g - M), O = sum_g o_g 2^(m_g - M) / L
  float M = -INFINITY;
  for (int g = 0; g < G; ++g) M = fmaxf(M, sm.s0[g]);
  float L = 0.f;
  for (int g = 0; g < G; ++g) L += sm.s1[g] * fast_exp2(sm.s0[g] - M);
  const int64_t lrow = (int64_t)plane * N + r;
  if (tid == 0) p.lse[lrow] = (M + fast_log2(L)) * kLn2;
  if (tid < D / 4) {
    float x[4] = {};
    for (int g = 0; g < G; ++g) {
      const float w = fast_exp2(sm.s0[g] - M);
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = __builtin_fmaf(sm.v0[g * D + 4 * tid + e], w, x[e]);
    }
    const float il = 1.f / L;
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] *= il;
    IO* O = const_cast<IO*>(plane_row<IO>(p.o, p.so, plane, p.H, r));
    store4(O + 4 * tid * p.so[3], p.so[3], p.vec_o, x);
    if constexpr (std::is_same<IO, bf16>::value) {
      if (p.o_res) {
        // rounding residual bf16(O - bf16(O)), contiguous [B, H, N, D]
        float res[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) res[e] = x[e] - (float)(bf16)x[e];
        store4(static_cast<bf16*>(p.o_res) + lrow * D + 4 * tid, 1, true, res);
      }
    }
  }
}

template <typename IO, int D, bool VEC>
__global__ void __launch_bounds__(kTailThreads) bwd_tail_rows_kernel(const BwdParams p, int row0,
                                                                      int write_delta) {
  constexpr int LPR = D / 8, G = kTailThreads / LPR;
  __shared__ TailLds<D> sm;
  const int tid = thread_id(), grp = tid / LPR, c = tid % LPR;
  const int N = p.N, R = N - row0, shift = 1 - p.has_cls;
  const int plane = block_id() / R, r = row0 + block_id() % R;
  const int64_t lrow = (int64_t)plane * N + r;

  float q[8], g[8];
  load_rot8<VEC, IO, D>(plane_row<IO>(p.q, p.sq, plane, p.H, r), p.sq, c, p.rope, r + shift, q);
#pragma unroll
  for (int e = 0; e < 8; ++e) q[e] *= p.scale_log2;
  load_row8<VEC>(plane_row<IO>(p.dout, p.sdo, plane, p.H, r), p.sdo, c, g);
  float delta;
  if (write_delta) {
    // delta = rowsum(dO * O), O plus its rounding residual when there is one
    float o[8];
    load_row8<VEC>(plane_row<IO>(p.o, p.so, plane, p.H, r), p.so, c, o);
    if constexpr (std::is_same<IO, bf16>::value) {
      if (p.o_res) {
        float x[8];
        unpack8(load_raw8(static_cast<const bf16*>(p.o_res) + lrow * D + 8 * c, 1, true), x);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += x[e];
      }
    }
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) d = __builtin_fmaf(g[e], o[e], d);
    delta = group_sum<LPR>(d);   // every group holds the same row
    if (tid == 0) p.delta[lrow] = delta;
  } else {
    delta = p.delta[lrow];
  }
  const float lse2 = p.lse[lrow] * kLog2e;

  float dq[8] = {};
  for (int j0 = grp; j0 < N; j0 += kTailU * G) {
    float k[kTailU][8], v[kTailU][8];
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      const int j = min(j0 + u * G, N - 1);
      load_rot8<VEC, IO, D>(plane_row<IO>(p.k, p.sk, plane, p.H, j), p.sk, c, p.rope, j + shift, k[u]);
      load_row8<VEC>(plane_row<IO>(p.v, p.sv, plane, p.H, j), p.sv, c, v[u]);
    }
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s = __builtin_fmaf(q[e], k[u][e], s);
        dp = __builtin_fmaf(g[e], v[u][e], dp);
      }
      s = group_sum<LPR>(s);
      dp = group_sum<LPR>(dp);
      const float ds = j0 + u * G < N ? fast_exp2(s - lse2) * (dp - delta) : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dq[e] = __builtin_fmaf(ds, k[u][e], dq[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) sm.v0[grp * D + 8 * c + e] = dq[e];
  __syncthreads();
  if (tid < D / 4) {
    float x[4] = {};
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] += sm.v0[gi * D + 4 * tid + e];
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] *= p.scale;
    rope_unrotate4(x, p.rope, r + shift, D / 2, 2 * tid);
    IO* DQ = const_cast<IO*>(plane_row<IO>(p.dq, p.sdq, plane, p.H, r));
    store4(DQ + 4 * tid * p.sdq[3], p.sdq[3], p.vec_dq, x);
  }
}

template <typename IO, int D, bool VEC>
__global__ void __launch_bounds__(kTailThreads) bwd_tail_keys_kernel(const BwdParams p, int key0) {
  constexpr int LPR = D / 8, G = kTailThreads / LPR;
  __shared__ TailLds<D> sm;
  const int tid = thread_id(), grp = tid / LPR, c = tid % LPR;
  const int N = p.N, R = N - key0, shift = 1 - p.has_cls;
  const int plane = block_id() / R, kc = key0 + block_id() % R;

  float k[8], v[8];
  load_rot8<VEC, IO, D>(plane_row<IO>(p.k, p.sk, plane, p.H, kc), p.sk, c, p.rope, kc + shift, k);
  load_row8<VEC>(plane_row<IO>(p.v, p.sv, plane, p.H, kc), p.sv, c, v);
  float ks[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) ks[e] = k[e] * p.scale_log2;

  float dk[8] = {}, dv[8] = {};
  const float* lse = p.lse + (int64_t)plane * N;
  const float* dl = p.delta + (int64_t)plane * N;
  for (int i0 = grp; i0 < N; i0 += kTailU * G) {
    float q[kTailU][8], g[kTailU][8], l2[kTailU], dl2[kTailU];
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      const int i = min(i0 + u * G, N - 1);
      load_rot8<VEC, IO, D>(plane_row<IO>(p.q, p.sq, plane, p.H, i), p.sq, c, p.rope, i + shift, q[u]);
      load_row8<VEC>(plane_row<IO>(p.dout, p.sdo, plane, p.H, i), p.sdo, c, g[u]);
      l2[u] = lse[i];
      dl2[u] = dl[i];
    }
#pragma unroll
    for (int u = 0; u < kTailU; ++u) {
      float s = 0.f, dp = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s = __builtin_fmaf(q[u][e], ks[e], s);
        dp = __builtin_fmaf(g[u][e], v[e], dp);
      }
      s = group_sum<LPR>(s);
      dp = group_sum<LPR>(dp);
      const float pr = i0 + u * G < N ? fast_exp2(s - l2[u] * kLog2e) : 0.f;
      const float ds = pr * (dp - dl2[u]);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dv[e] = __builtin_fmaf(pr, g[u][e], dv[e]);
        dk[e] = __builtin_fmaf(ds, q[u][e], dk[e]);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    sm.v0[grp * D + 8 * c + e] = dk[e];
    sm.v1[grp * D + 8 * c + e] = dv[e];
  }
  __syncthreads();
  if (tid < D / 4) {
    float xk[4] = {}, xv[4] = {};
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xk[e] += sm.v0[gi * D + 4 * tid + e];
        xv[e] += sm.v1[gi * D + 4 * tid + e];
      }
#pragma unroll
    for (int e = 0; e < 4; ++e) xk[e] *= p.scale;
    rope_unrotate4(xk, p.rope, kc + shift, D / 2, 2 * tid);
    IO* DK = const_cast<IO*>(plane_row<IO>(p.dk, p.sdk, plane, p.H, kc));
    IO* DV = const_cast<IO*>(plane_row<IO>(p.dv, p.sdv, plane, p.H, kc));
    store4(DK + 4 * tid * p.sdk[3], p.sdk[3], p.vec_dk, xk);
    store4(DV + 4 * tid * p.sdv[3], p.sdv[3], p.vec_dv, xv);
  }
}

// The plane's last key when the dQ kernel summed its dK-hat / dV rows per
// query tile (p.xk_ws: nparts row pairs per plane, dK-hat then dV): the
// tiles' rows added in order, dK-hat scaled and rotated back, both stored.
// One workgroup per plane, D/4 threads of 4 channels.
template <typename IO, int D>
__global__ void __launch_bounds__(D / 4) bwd_tail_key_merge_kernel(const BwdParams p, int nparts) {
  const int plane = block_id(), tid = thread_id();
  const int N = p.N, kc = N - 1, shift = 1 - p.has_cls;
  const float* w = p.xk_ws + (int64_t)plane * nparts * (2 * D);
  float xk[4] = {}, xv[4] = {};
  for (int b = 0; b < nparts; ++b)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xk[e] += w[b * 2 * D + 4 * tid + e];
      xv[e] += w[b * 2 * D + D + 4 * tid + e];
    }
#pragma unroll
  for (int e = 0; e < 4; ++e) xk[e] *= p.scale;
  rope_unrotate4(xk, p.rope, kc + shift, D / 2, 2 * tid);
  IO* DK = const_cast<IO*>(plane_row<IO>(p.dk, p.sdk, plane, p.H, kc));
  IO* DV = const_cast<IO*>(plane_row<IO>(p.dv, p.sdv, plane, p.H, kc));
  store4(DK + 4 * tid * p.sdk[3], p.sdk[3], p.vec_dk, xk);
  store4(DV + 4 * tid * p.sdv[3], p.sdv[3], p.vec_dv, xv);
}

template <typename IO, bool VEC>
hipError_t fwd_tail_v(const FwdParams& p, int D, int row0, hipStream_t st) {
  const dim3 grid(p.B * p.H * (p.N - row0)), block(kTailThreads);
  switch (D) {
    case 32: hipLaunchKernelGGL((fwd_tail_kernel<IO, 32, VEC>), grid, block, 0, st, p, row0); break;
    case 64: hipLaunchKernelGGL((fwd_tail_kernel<IO, 64, VEC>), grid, block, 0, st, p, row0); break;
    case 128: hipLaunchKernelGGL((fwd_tail_kernel<IO, 128, VEC>), grid, block, 0, st, p, row0); break;
    case 256: hipLaunchKernelGGL((fwd_tail_kernel<IO, 256, VEC>), grid, block, 0, st, p, row0); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename IO, bool VEC>
hipError_t rows_tail_v(const BwdParams& p, int D, int row0, int write_delta, hipStream_t st) {
  const dim3 grid(p.B * p.H * (p.N - row0)), block(kTailThreads);
  switch (D) {
    case 32: hipLaunchKernelGGL((bwd_tail_rows_kernel<IO, 32, VEC>), grid, block, 0, st, p, row0, write_delta); break;
    case 64: hipLaunchKernelGGL((bwd_tail_rows_kernel<IO, 64, VEC>), grid, block, 0, st, p, row0, write_delta); break;
    case 128: hipLaunchKernelGGL((bwd_tail_rows_kernel<IO, 128, VEC>), grid, block, 0, st, p, row0, write_delta); break;
    case 256: hipLaunchKernelGGL((bwd_tail_rows_kernel<IO, 256, VEC>), grid, block, 0, st, p, row0, write_delta); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename IO, bool VEC>
hipError_t keys_tail_v(const BwdParams& p, int D, int key0, hipStream_t st) {
  const dim3 grid(p.B * p.H * (p.N - key0)), block(kTailThreads);
  switch (D) {
    case 32: hipLaunchKernelGGL((bwd_tail_keys_kernel<IO, 32, VEC>), grid, block, 0, st, p, key0); break;
    case 64: hipLaunchKernelGGL((bwd_tail_keys_kernel<IO, 64, VEC>), grid, block, 0, st, p, key0); break;
    case 128: hipLaunchKernelGGL((bwd_tail_keys_kernel<IO, 128, VEC>), grid, block, 0, st, p, key0); break;
    case 256: hipLaunchKernelGGL((bwd_tail_keys_kernel<IO, 256, VEC>), grid, block, 0, st, p, key0); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// vector loads when every row the kernel reads allows them
template <typename IO>
hipError_t fwd_tail_d(const FwdParams& p, int D, int row0, hipStream_t st) {
  return p.vec_q && p.vec_k && p.vec_v ? fwd_tail_v<IO, true>(p, D, row0, st)
                                       : fwd_tail_v<IO, false>(p, D, row0, st);
}

template <typename IO>
hipError_t rows_tail_d(const BwdParams& p, int D, int row0, int write_delta, hipStream_t st) {
  const bool vec = p.vec_q && p.vec_k && p.vec_v && p.vec_do && (!write_delta || p.vec_o);
  return vec ? rows_tail_v<IO, true>(p, D, row0, write_delta, st)
             : rows_tail_v<IO, false>(p, D, row0, write_delta, st);
}

template <typename IO>
hipError_t keys_tail_d(const BwdParams& p, int D, int key0, hipStream_t st) {
  return p.vec_q && p.vec_k && p.vec_v && p.vec_do ? keys_tail_v<IO, true>(p, D, key0, st)
                                                   : keys_tail_v<IO, false>(p, D, key0, st);
}

}  // namespace

int tail_rows(int N, int block_rows) {
  const int r = N % block_rows;
  return (N >= block_rows && r > 0 && r <= kTailMaxRows) ? r : 0;
}

hipError_t launch_fwd_tail(const FwdParams& p, int io, int D, int row0, hipStream_t st) {
  switch (io) {
    case DT_BF16: return fwd_tail_d<bf16>(p, D, row0, st);
    case DT_F16: return fwd_tail_d<f16>(p, D, row0, st);
    default: return fwd_tail_d<float>(p, D, row0, st);
  }
}

hipError_t launch_bwd_tail_rows(const BwdParams& p, int io, int D, int row0, bool write_delta,
                                hipStream_t st) {
  switch (io) {
    case DT_BF16: return rows_tail_d<bf16>(p, D, row0, write_delta, st);
    case DT_F16: return rows_tail_d<f16>(p, D, row0, write_delta, st);
    default: return rows_tail_d<float>(p, D, row0, write_delta, st);
  }
}

hipError_t launch_bwd_tail_key_merge(const BwdParams& p, int io, int D, int nparts, hipStream_t st) {
  const dim3 grid(p.B * p.H);
  if (io != DT_BF16 && io != DT_F16) return hipErrorInvalidValue;
  if (D == 128) {
    if (io == DT_BF16) hipLaunchKernelGGL((bwd_tail_key_merge_kernel<bf16, 128>), grid, dim3(32), 0, st, p, nparts);
    else hipLaunchKernelGGL((bwd_tail_key_merge_kernel<f16, 128>), grid, dim3(32), 0, st, p, nparts);
  } else if (D == 256) {
    if (io == DT_BF16) hipLaunchKernelGGL((bwd_tail_key_merge_kernel<bf16, 256>), grid, dim3(64), 0, st, p, nparts);
    else hipLaunchKernelGGL((bwd_tail_key_merge_kernel<f16, 256>), grid, dim3(64), 0, st, p, nparts);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bwd_tail_keys(const BwdParams& p, int io, int D, int key0, hipStream_t st) {
  switch (io) {
    case DT_BF16: return keys_tail_d<bf16>(p, D, key0, st);
    case DT_F16: return keys_tail_d<f16>(p, D, key0, st);
    default: return keys_tail_d<float>(p, D, key0, st);
  }
}

}  // namespace farope
