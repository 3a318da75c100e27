// Forward kernel: O = softmax(scale * (R Q)(R K)^T) V and LSE, fused 2D RoPE.
//
// Reference behaviour followed: _attn_fwd in "fa_rope_full .py" (FA:91-315):
// Q/K pair rotation with the CLS row bypassing RoPE (FA:176-202, FA:248-272),
// scaled logits with padded key columns masked out (FA:275-277), online
// softmax with a running max (FA:280-305) and the per-row log-sum-exp stored
// for the backward pass (FA:308-309).
//
// gfx950 design:
//  * Persistent workgroups.  A work item is (b, h) plane x block of
//    NW*QT*16 query rows (one item per plane when N <= 256 at D = 64).  Each
//    workgroup walks its items with ONE continuous software pipeline: the next
//    KV chunk -- of this item, or the first chunk of the next item -- is in
//    flight in registers while the current chunk is computed, and the next
//    item's Q rows are loaded while the current item runs.  HBM latency is
//    therefore hidden behind compute even at one workgroup per CU.
//  * Wave w owns q-subtiles w, w+NW, ... (16 rows each) of the item, so the
//    ragged tail (N = 1 + H_img^2) is spread over the waves.  Rotated Q rows
//    stay in registers as MFMA B-operands.
//  * K and V go through a 2-slot LDS ring of KC-key chunks.  K is rotated in
//    fp32 on its way in (row-major K-hat, rows permuted so the 16 rows one
//    MFMA reads are consecutive: no bank conflicts); V is stored transposed,
//    two keys per 32-bit LDS write.  The ragged chunk of a plane is processed
//    first, so the cross-item prefetch always overlaps a full chunk.
//  * Logits are computed transposed, S^T = K-hat Q-hat^T, with key
//    kv = 8*(r/4) + 4*h + r%4 of a 32-key block in A-row r of half h.  Lane
//    group lg then holds keys 8*lg .. 8*lg+7 of its query column: exactly the
//    B-operand of O^T += V^T P^T, so P never leaves registers and each K-hat /
//    V^T fragment (one 16-byte LDS read) feeds all QT subtiles of the wave.
//  * One query row per lane: the row max needs two cross-lane steps per
//    32-key block.  Softmax runs in base 2 (log2(e) folded into the scale)
//    with fp32 state and accumulator; O and the row sum are rescaled only
//    when the running max grows by more than 2^8 (P <= 256 otherwise).
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

// V^T tile: the 8-key group g of channel row d is stored at group
// g ^ ((d >> 3) & 7).  With a row pitch of KC + 16 elements this makes both
// the transposed stores (8 channel rows x 2 key pairs per 16 lanes) and the
// MFMA fragment reads (16 channel rows, one group) bank-conflict free.
__device__ __forceinline__ int vswz(int d, int col) {
  return (((col >> 3) ^ ((d >> 3) & 7)) << 3) | (col & 7);
}

constexpr float kRescaleSlack = 8.0f;   // log2 units: P <= 2^8 between rescales

// VEC: every tensor of the call allows 16-byte vector access (decided on the
// host); the generic instantiation gathers element by element instead.
// FS (bf16 compute): the logits product takes fp16 operands (K-hat tile in
// LDS, Q-hat fragments in registers): the rounding of the rotated rows to
// bf16 is what dominates the error of bf16 attention at long, wide planes.
// O = P V takes fp16 P and V too (V times fv; bf16 values convert exactly
// inside fp16's range): with bf16 P, O's computation error (2^-9 per
// probability) was as large as its storage rounding, and the backward's
// delta = rowsum(dO * O) inherits it.  An item whose Q-hat or K-hat reaches
// 2^12, or whose V leaves [2^-10, 2^12), is computed again with scaled
// operands (f16_fit in common.h).
template <typename IO, int CT, int D, int NW, int QT, int KC, int TABROWS, bool VEC, bool FS>
__global__ void __launch_bounds__(NW * 64)
fwd_kernel(const FwdParams p) {
  using C = Comp<CT>;
  using S = typename C::S;
  using Frag = typename C::Frag;
  using LC = std::conditional_t<FS, Comp<DT_F16>, C>;   // logits operands
  using LFrag = typename LC::Frag;
  using VC = std::conditional_t<FS, Comp<DT_F16>, C>;   // P and V operands
  using VS = typename VC::S;
  using VFrag = typename VC::Frag;
  constexpr int KS = D / 32;          // k-steps of 32 channels
  constexpr int DT = D / 16;          // 16-channel output subtiles
  constexpr int D2 = D / 2;
  // K-hat / V row padding: 16 bytes, or 32 with fp16 logits at D >= 128 (the
  // pitch at which 16-byte reads of 16 consecutive rows, the K-hat fragment
  // reads, measured conflict-free in isolation; HiRes forward -2 us)
  constexpr int PADE = (FS && D >= 128) ? 16 : 16 / sizeof(S);
  constexpr int LDK = D + PADE;       // K-hat row pitch (elements)
  constexpr int LDV = KC + 16;        // V^T row pitch (elements; see vswz)
  constexpr int NT = NW * 64;
  constexpr int CPR = D / 8;          // 8-channel chunks per row
  constexpr int UNITS = (KC / 2) * CPR;   // (row pair, chunk) staging units per KV chunk
  constexpr int ITER = (UNITS + NT - 1) / NT;
  static_assert(KC % 32 == 0, "KV chunk must be a multiple of 32 keys");
  // TABROWS > 0: the whole packed RoPE table (<= TABROWS rows) is copied into
  // LDS once per persistent workgroup and all rotations read it from there;
  // TABROWS == 0: rotations read the table from global memory (L2-resident).
  constexpr bool kTabLds = TABROWS > 0;

  // 16-bit compute: V is kept row-major (raw rows when IO is the compute
  // type) and V^T fragments are read transposed (ds_read_b64_tr_b16); fp32
  // compute keeps an explicitly transposed V^T tile, except at D = 256, where
  // two transposed fp32 tiles do not fit next to the K-hat ring: V stays
  // row-major and each V^T fragment is gathered element by element (VROW).
  constexpr bool TRV = sizeof(S) == 2;
  constexpr bool VROW = !TRV && D >= 256;
  static_assert(!FS || CT == DT_BF16, "fp16 logit operands go with bf16 compute");
  __shared__ __attribute__((aligned(16))) S sK[2][KC * LDK];   // FS: fp16 K-hat
  // FS: per-wave max |Q-hat|, max |K-hat| bit patterns of an item pass
  __shared__ u32x4 sRange[FS ? NW : 1];
  __shared__ __attribute__((aligned(16))) VS sVt[2][(TRV || VROW) ? KC * LDK : D * LDV];
  // XR: the plane's last row, when it is the only one past the full query
  // blocks (p.x_rows == 1, N = 1 + a multiple of the block rows), rides along
  // one designated item of the plane instead of a tail kernel that would read
  // the whole plane's K and V again.  Its logits and O run on the VALU against
  // the same staged K-hat / V chunks: wave w takes keys KC/NW * w .. of each
  // chunk, keeps its own online-softmax state in LDS, and the NW partial
  // states merge at the item's end.  Its Q-hat row is staged like the others
  // (fp16, scaled by c2 * fq, counted in the operand range).
  constexpr bool XR = FS && VEC && sizeof(IO) == 2 && KC == 8 * NW;
  constexpr int XO = XR ? D / 64 : 1;  // output channels per lane (XR)
  __shared__ __attribute__((aligned(16))) f16 sXq[XR ? 2 : 1][XR ? D : 8];   // by pass parity
  __shared__ __attribute__((aligned(16))) float sXo[XR ? NW : 1][XR ? D : 4];
  __shared__ float sXml[XR ? NW : 1][2];
  // LDS copy of the packed table: D/2 (cos, sin) pairs = D floats per row,
  // 16-byte chunk c of row r stored at chunk c ^ (r & (D/4 - 1)) (bank-spread
  // without padding).
  constexpr int TCH = D / 4;          // 16-byte chunks per table row (D floats)
  __shared__ __attribute__((aligned(16))) float sTab[kTabLds ? TABROWS * 2 * D / 2 : 4];

  const int N = p.N;
  const int nch = (N + KC - 1) / KC;  // KV chunks per item
  const bool vec_q = VEC || p.vec_q, vec_k = VEC || p.vec_k;
  const bool vec_v = VEC || p.vec_v, vec_o = VEC || p.vec_o;
  const int shift = 1 - p.has_cls;    // table row of token s is s + shift
  const float c2 = p.scale_log2;
  // cos/sin of pairs p0 .. p0+3 of table row `row`.
  auto tab4 = [&](int row, int p0, float (&cs)[8]) __attribute__((always_inline)) {
    if constexpr (kTabLds) {
      const int c = p0 >> 1;   // chunks c, c + 1 hold pairs p0 .. p0+3
      const f32x4 a = *reinterpret_cast<const f32x4*>(&sTab[(row * TCH + (c ^ (row & (TCH - 1)))) * 4]);
      const f32x4 b = *reinterpret_cast<const f32x4*>(&sTab[(row * TCH + ((c + 1) ^ (row & (TCH - 1)))) * 4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        cs[e] = a[e];
        cs[4 + e] = b[e];
      }
    } else {
      rope_load4(p.rope, row, D2, p0, cs);
    }
  };

  const int tid = thread_id();
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
  const int lane = tid & 63;
  const int lr = lane & 15, lg = lane >> 4;
  // V tile rows of the lane's two transposed reads per 32-key block (see
  // vperm; key order where the two row constants would not fit the generic
  // D = 128 path's registers)
  constexpr bool kVperm = sizeof(S) == 2 && (VEC || D <= 64);
  auto vrow = [](int r) { return kVperm ? vperm(r) : r; };
  const int vr0 = vrow(8 * lg + (lr >> 2)), vr1 = vrow(8 * lg + 4 + (lr >> 2));

  // Item of this workgroup at iteration `it` (-1 when done).  Within an
  // iteration, items are dealt XCD-major so neighbouring items (the q blocks
  // of one plane) run on the same XCD and share its L2.
  const int pos = xcd_remap(block_id(), p.n_wg);
  auto item_of = [&](int it) __attribute__((always_inline)) {
    const int item = it * p.n_wg + pos;
    return item < p.n_items ? item : -1;
  };
  auto plane_base = [&](const void* base, const int64_t* st, int plane) __attribute__((always_inline)) {
    const int bb = plane / p.H, hh = plane - bb * p.H;
    return static_cast<const IO*>(base) + bb * st[0] + hh * st[1];
  };
  // Chunk c of an item starts at key ((c + nch - 1) % nch) * KC: ragged chunk first.
  auto chunk_start = [&](int c) __attribute__((always_inline)) { return ((c + nch - 1) % nch) * KC; };

  // VEC: the host guarantees unit d-stride, 16-byte alignment and in-plane
  // byte offsets below 2^31.  Prefetches then go through buffer descriptors
  // over rows 0 .. N-1 of the plane: unconditional (rows >= N read 0), with
  // 32-bit lane byte offsets, so the wait-count pass can track each prefetch
  // precisely instead of draining all outstanding loads at control-flow joins.
  constexpr unsigned ES = sizeof(IO);
  auto rsrc = [&](const void* b, const int64_t* st, int plane) __attribute__((always_inline)) {
    return make_rsrc(plane_base(b, st, plane), (unsigned)(((int64_t)(N - 1) * st[2] + D) * ES));
  };

  // FS: largest |Q-hat| (scaled) and |K-hat| this thread converted in the
  // current pass of an item; the operand scales and the logit factor
  // 1 / (fq fk) of a rescaled pass (all 1 otherwise).
  float amax_q = 0.f, amax_k = 0.f;
  float amax_vf = 0.f;       // FS: largest |V * fv| of the pass
  float fq = 1.f, fk = 1.f, fsc = 1.f, fv = 1.f;
  float ifv = 1.f;   // 1 / fv of the item's kept pass (O comes out times fv)
  bool rescaled = false, redo = false;
  unsigned eq = 0, ek = 0, ev = 0;   // biased exponents of the pass's max |Q-hat|, |K-hat|, |V|

  // ---- KV chunk prefetch registers: two rows x 8 channels of K and V
  //      (+ their cos/sin when the table is not in LDS) ----
  Raw8<IO> pk[ITER][2], pv[ITER][2];
  float pcs[ITER][2][kTabLds ? 1 : 8];
  // K / V buffer descriptors of one item's plane (SGPRs), built once per item
  // -- in the previous item's last chunk, whose prefetch is the first to read
  // the item -- instead of per chunk (the plane split and the 64-bit base
  // arithmetic are most of a chunk's scalar work).  Used when every wave
  // loads whole units (UNITS a multiple of the workgroup size).
  struct KvRs {
    __amdgpu_buffer_rsrc_t k, v;
  };
  auto kv_rs = [&](int item) __attribute__((always_inline)) {
    const int plane = item / p.n_blk;
    return KvRs{rsrc(p.k, p.sk, plane), rsrc(p.v, p.sv, plane)};
  };
  auto prefetch_kv = [&](int item, const KvRs& kr, int c) __attribute__((always_inline)) {
    const int plane = item / p.n_blk;
    if constexpr (VEC && kTabLds && UNITS % NT == 0) {
      const int kvb = chunk_start(c);
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int u = tid + it * NT;
        const int rp = u / CPR, cc = u - rp * CPR;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int r = 2 * rp + x;
          pk[it][x] = buf_load8<IO>(kr.k, (unsigned)((r * (int)p.sk[2] + 8 * cc) * (int)ES),
                                    (unsigned)(kvb * (int)p.sk[2] * (int)ES));
          pv[it][x] = buf_load8<IO>(kr.v, (unsigned)((r * (int)p.sv[2] + 8 * cc) * (int)ES),
                                    (unsigned)(kvb * (int)p.sv[2] * (int)ES));
        }
      }
      return;
    }
    if constexpr (VEC && !kTabLds && UNITS % NT == 0) {
      // table rows from global memory too, through a descriptor over rows
      // 0 .. N-1+shift: per-lane offsets fixed across chunks, the chunk's row
      // in the uniform offset; rows >= N (zero K rows) read zeros
      const int kvb = chunk_start(c);
      const auto rT = make_rsrc(p.rope, (unsigned)((N + shift) * D * 4));
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int u = tid + it * NT;
        const int rp = u / CPR, cc = u - rp * CPR;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int r = 2 * rp + x;
          pk[it][x] = buf_load8<IO>(kr.k, (unsigned)((r * (int)p.sk[2] + 8 * cc) * (int)ES),
                                    (unsigned)(kvb * (int)p.sk[2] * (int)ES));
          pv[it][x] = buf_load8<IO>(kr.v, (unsigned)((r * (int)p.sv[2] + 8 * cc) * (int)ES),
                                    (unsigned)(kvb * (int)p.sv[2] * (int)ES));
          const unsigned to = (unsigned)(((r + shift) * D + 8 * cc) * 4);
          const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rT, to, (unsigned)(kvb * D * 4), 0);
          const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rT, to + 16, (unsigned)(kvb * D * 4), 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            pcs[it][x][e] = __uint_as_float(a[e]);
            pcs[it][x][4 + e] = __uint_as_float(b[e]);
          }
        }
      }
      return;
    }
    if constexpr (VEC && kTabLds && UNITS % 64 == 0) {
      // every wave loads whole units or none (UNITS is a multiple of the wave
      // size): a wave without a unit gets empty-range descriptors, so its
      // loads stay unconditional and return zeros without memory traffic
      const int kvb = chunk_start(c);
#pragma unroll
      for (int it = 0; it < ITER; ++it) {
        const int u0 = tid + it * NT;
        const bool act = UNITS % NT == 0 || u0 < UNITS;   // wave-uniform
        const int u = act ? u0 : 0;
        const auto rK = make_rsrc(plane_base(p.k, p.sk, plane), act ? (unsigned)(((int64_t)(N - 1) * p.sk[2] + D) * ES) : 0u);
        const auto rV = make_rsrc(plane_base(p.v, p.sv, plane), act ? (unsigned)(((int64_t)(N - 1) * p.sv[2] + D) * ES) : 0u);
        const int rp = u / CPR, cc = u - rp * CPR;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
          const int r = 2 * rp + x;
          pk[it][x] = buf_load8<IO>(rK, (unsigned)((r * (int)p.sk[2] + 8 * cc) * (int)ES),
                                    (unsigned)(kvb * (int)p.sk[2] * (int)ES));
          pv[it][x] = buf_load8<IO>(rV, (unsigned)((r * (int)p.sv[2] + 8 * cc) * (int)ES),
                                    (unsigned)(kvb * (int)p.sv[2] * (int)ES));
        }
      }
      return;
    }
    const IO* __restrict__ K = plane_base(p.k, p.sk, plane);
    const IO* __restrict__ V = plane_base(p.v, p.sv, plane);
    const int kvb = chunk_start(c);
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
          if constexpr (!kTabLds) rope_load4(p.rope, gr + shift, D2, 4 * cc, pcs[it][x]);
        } else {
          pk[it][x] = zero_raw8<IO>();
          pv[it][x] = zero_raw8<IO>();
          if constexpr (!kTabLds) {
#pragma unroll
            for (int e = 0; e < 8; ++e) pcs[it][x][e] = 0.f;
          }
        }
      }
    }
  };
  auto commit_kv = [&](int slot, int kvb) __attribute__((always_inline)) {
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
          if constexpr (kTabLds) {
            // rows past N hold zeros; any in-table row serves for them
            float cs[8];
            tab4(min(kvb + 2 * rp + x, N - 1) + shift, 4 * cc, cs);
            rope_rotate8(xk, cs);
          } else {
            rope_rotate8(xk, pcs[it][x]);
          }
          // K-hat pre-scaled by softmax_scale * log2(e): the logits come out
          // of the MFMAs in log2 units (every kernel stages K-hat this way, so
          // the forward and backward passes see bit-identical logits).  With
          // fp16 operands Q-hat carries the scale instead (in every kernel):
          // it is staged once per item, K-hat once per chunk.
          if constexpr (!FS) {
#pragma unroll
            for (int e = 0; e < 8; ++e) xk[e] *= c2;
          }
          if constexpr (FS) {
            if (rescaled) {
#pragma unroll
              for (int e = 0; e < 8; ++e) xk[e] *= fk;
            }
            amax_k = opaque(amax8(amax_k, xk));   // (computed here, not at the item's end)
            *reinterpret_cast<f16x8*>(&sK[slot][kperm(2 * rp + x) * LDK + 8 * cc]) = to_f16x8(xk);
          } else {
            C::put8(&sK[slot][kperm(2 * rp + x) * LDK + 8 * cc], xk);
          }
          if constexpr (FS) {
            // V in fp16, times fv (1 except in a rescaled pass, which alone
            // multiplies); its range from the converted values
            float y[8];
            unpack8(pv[it][x], y);
            if (rescaled) {
#pragma unroll
              for (int e = 0; e < 8; ++e) y[e] *= fv;
            }
            amax_vf = opaque(amax8(amax_vf, y));
            *reinterpret_cast<f16x8*>(&sVt[slot][vrow(2 * rp + x) * LDK + 8 * cc]) = to_f16x8(y);
          } else if constexpr (TRV || VROW) {
            S* dst = &sVt[slot][vrow(2 * rp + x) * LDK + 8 * cc];
            if constexpr (std::is_same<IO, S>::value) {
              *reinterpret_cast<typename Raw8<IO>::vec*>(dst) = pv[it][x].v;   // raw row segment
            } else {
              float y[8];
              unpack8(pv[it][x], y);
              C::put8(dst, y);
            }
          } else {
            unpack8(pv[it][x], xv[x]);
          }
        }
        if constexpr (!TRV && !VROW) {
#pragma unroll
          for (int e = 0; e < 8; ++e)
            put2<CT>(&sVt[slot][(8 * cc + e) * LDV + vswz(8 * cc + e, 2 * rp)], xv[0][e], xv[1][e]);
        }
      }
    }
  };

  // ---- Q rows of an item: raw prefetch registers -> rotated B-operand fragments ----
  // At D = 128 with two subtiles per wave, or with fp16 logit operands, the
  // rows load when the item starts instead: the prefetch registers (rows and
  // table values) would not fit beside the Q-hat fragments and O
  // accumulators, and an item computed again (fp16 operand range) needs its
  // own rows.
  constexpr bool kQpf = !(FS || (D == 128 && QT > 1));
  Raw8<IO> qraw[kQpf ? QT : 1][kQpf ? KS : 1];
  float qcs[kQpf ? QT : 1][kQpf ? KS : 1][kTabLds ? 1 : 8];
  auto prefetch_q = [&](int item) __attribute__((always_inline)) {
    if constexpr (!kQpf) return;
    const int plane = item / p.n_blk, qb = item - plane * p.n_blk;
    if constexpr (VEC && kTabLds) {
      const auto rQ = rsrc(p.q, p.sq, plane);
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
#pragma unroll
        for (int s = 0; s < KS; ++s)
          qraw[t][s] = buf_load8<IO>(rQ, (unsigned)((row * (int)p.sq[2] + 32 * s + 8 * lg) * (int)ES), 0u);
      }
      return;
    }
    const IO* __restrict__ Q = plane_base(p.q, p.sq, plane);
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int c0 = 32 * s + 8 * lg;
        if (row < N) {
          qraw[t][s] = load_raw8(Q + row * p.sq[2] + c0 * p.sq[3], p.sq[3], vec_q);
          if constexpr (!kTabLds) rope_load4(p.rope, row + shift, D2, c0 / 2, qcs[t][s]);
        } else {
          qraw[t][s] = zero_raw8<IO>();
          if constexpr (!kTabLds) {
#pragma unroll
            for (int e = 0; e < 8; ++e) qcs[t][s][e] = 0.f;
          }
        }
      }
    }
  };
  LFrag qf[QT][KS];
  bool xi = false;   // XR: this item pass also computes the plane's last row
  // Q rows loaded at the item start (!kQpf) with vector access: through
  // descriptors over the plane's rows (rows >= N read 0; lanes with no part
  // of the plane's last row read past the range), every load of the item's
  // Q-hat fragments, their table values and (XR) the plane's last row goes
  // out before the first is used, so the item start waits once for all of
  // them (a load per fragment behind a row test waited once per fragment,
  // each time also for every store still in flight).
  constexpr bool kQdesc = !kQpf && VEC;
  Raw8<IO> qld[kQdesc ? QT : 1][kQdesc ? KS : 1];
  float qtb[kQdesc ? QT : 1][kQdesc ? KS : 1][kQdesc ? 8 : 1];
  Raw8<IO> xld;
  float xtb[8];
  auto load_q = [&](int plane, int qb) __attribute__((always_inline)) {
    if constexpr (kQdesc) {
      const auto rQ = rsrc(p.q, p.sq, plane);
      const auto rT = make_rsrc(p.rope, (unsigned)((N + shift) * D * 4));
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const int c0 = 32 * s + 8 * lg;
          qld[t][s] = buf_load8<IO>(rQ, (unsigned)((row * (int)p.sq[2] + c0) * (int)ES), 0u);
          const unsigned to = (unsigned)(((row + shift) * D + c0) * 4);
          const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rT, to, 0u, 0);
          const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rT, to + 16, 0u, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            qtb[t][s][e] = __uint_as_float(a[e]);
            qtb[t][s][4 + e] = __uint_as_float(b[e]);
          }
        }
      }
      if constexpr (XR) {
        const bool xl = wave == 0 && lane < D / 8;
        xld = buf_load8<IO>(rQ, xl ? (unsigned)(((N - 1) * (int)p.sq[2] + 8 * lane) * (int)ES) : 0x80000000u, 0u);
        const unsigned to = xl ? (unsigned)(((N - 1 + shift) * D + 8 * lane) * 4) : 0x80000000u;
        const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(rT, to, 0u, 0);
        const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(rT, to + 16u, 0u, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xtb[e] = __uint_as_float(a[e]);
          xtb[4 + e] = __uint_as_float(b[e]);
        }
      }
    }
  };
  int npass = 0;     // item passes so far (a rescaled pass counts again)
  auto commit_q = [&](int plane, int qb) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        float x[8];
        if constexpr (kQdesc) {
          unpack8(qld[t][s], x);
          rope_rotate8(x, qtb[t][s]);
        } else if constexpr (!kQpf) {
          const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
          const int c0 = 32 * s + 8 * lg;
          float cs[8];
          if (row < N) {
            unpack8(load_raw8(plane_base(p.q, p.sq, plane) + row * p.sq[2] + c0 * p.sq[3], p.sq[3], vec_q), x);
            rope_load4(p.rope, row + shift, D2, c0 / 2, cs);
            rope_rotate8(x, cs);
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = 0.f;
          }
        } else {
        unpack8(qraw[t][s], x);
        if constexpr (kTabLds) {
          const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
          float cs[8];
          tab4(min(row, N - 1) + shift, 16 * s + 4 * lg, cs);
          rope_rotate8(x, cs);
        } else {
          rope_rotate8(x, qcs[t][s]);
        }
        }
        if constexpr (FS) {
          const float qs = c2 * fq;
#pragma unroll
          for (int e = 0; e < 8; ++e) x[e] *= qs;
          amax_q = amax8(amax_q, x);
          qf[t][s].v = to_f16x8(x);
        } else {
          qf[t][s] = C::make(x);
        }
      }
    if constexpr (XR) {
      if (xi && wave == 0 && lane < D / 8) {
        static_assert(kQdesc, "the last row rides along vector-access items only");
        const int c0 = 8 * opaque(lane);
        float x[8];
        unpack8(xld, x);   // (row N - 1, channels c0 .. c0 + 7)
        rope_rotate8(x, xtb);
        const float qs = c2 * fq;
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] *= qs;
        amax_q = amax8(amax_q, x);
        *reinterpret_cast<f16x8*>(&sXq[npass & 1][c0]) = to_f16x8(x);
      }
    }
  };
  // XR: the last row against keys kvb + 8 * wave + (0..7) of a staged chunk.
  // Lane (key kk = lane / 8, slice ds = lane % 8) forms the fp16 dot product
  // over channels D/8 * ds .. of its key; then every lane updates channels
  // XO * lane .. of the wave's partial O with the 8 probabilities.
  auto xrow_chunk = [&](const S* __restrict__ cK, const VS* __restrict__ cV, int kvb, bool first)
      __attribute__((always_inline)) {
    // (lane addresses from an opaque copy: recomputed here, not kept live
    // through the chunk loop)
    const int ln = opaque(lane);
    const int kk = ln >> 3, ds = ln & 7;
    const int r = 8 * wave + kk;
    const f16* kp = reinterpret_cast<const f16*>(cK) + kperm(r) * LDK + (D / 8) * ds;
    const f16* qp = &sXq[npass & 1][(D / 8) * ds];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < D / 64; ++i)
      s = dot8<f16>(*reinterpret_cast<const Raw8<f16>*>(qp + 8 * i), *reinterpret_cast<const Raw8<f16>*>(kp + 8 * i), s);
    s = dpp_sum8(s);
    s = kvb + r < N ? s * fsc : -INFINITY;
    // the wave's 8 keys sit 8 lanes apart: row rotation by 8, then the row swaps
    float cm = fmaxf(s, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s), 0x128, 0xF, 0xF, false)));
    cm = group4_max(cm);
    const float mo = first ? -INFINITY : sXml[wave][0];
    const float lo = first ? 0.f : sXml[wave][1];
    const float mn = fmaxf(mo, cm);
    const float mb = mn == -INFINITY ? 0.f : mn;   // no valid key yet: all terms stay 0
    const float al = fast_exp2(mo - mb);
    const float pk = fast_exp2(s - mb);
    float ps = pk + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(pk), 0x128, 0xF, 0xF, false));
    ps = group4_sum(ps);
    float o[XO];
#pragma unroll
    for (int i = 0; i < XO; ++i) o[i] = first ? 0.f : sXo[wave][XO * ln + i] * al;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float pj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pk), 8 * j));
      const VS* vp = cV + vrow(8 * wave + j) * LDK + XO * ln;
#pragma unroll
      for (int i = 0; i < XO; ++i) o[i] = __builtin_fmaf(pj, (float)vp[i], o[i]);
    }
#pragma unroll
    for (int i = 0; i < XO; ++i) sXo[wave][XO * ln + i] = o[i];
    if (ln == 0) {
      sXml[wave][0] = mn;
      sXml[wave][1] = __builtin_fmaf(lo, al, ps);
    }
  };

  float m_run[QT], l_run[QT], m_thr[QT];
  // Pipelined chunks (kPipe): the logits accumulators of a block start at
  // -mb (mb = m_run once it is finite, else 0), so the MFMAs deliver
  // S - m_run and P = exp2(acc) needs no subtraction; m_thr then holds the
  // threshold relative to mb.
  float mb[QT];
  f32x4 oacc[QT][DT];

  // The 32-key blocks of a KV chunk run as a software pipeline over all QT
  // subtiles of the wave.  Step j issues the LDS reads of block j+1's K-hat
  // fragments and block j's V^T fragments, runs the softmax of block j on the
  // VALU while the MFMA pipe still computes block j's logits, then issues the
  // logits of block j+1 and O^T += V^T P^T of block j.  Subtiles past the last
  // query row hold zero rows and are computed anyway: every wave of a
  // workgroup then runs the same instruction stream with no per-subtile
  // guards, and for the 16-row-ragged N of ViT planes the extra work lands on
  // SIMDs that would otherwise wait at the next barrier.
  // VROW: V^T fragment (rows 16d.., k-slot e <-> key 32j + 8lg + e) gathered
  // from the row-major V tile, one element per key row.
  auto vrow_frag = [&](const VS* __restrict__ cV, int j, int d) __attribute__((always_inline)) {
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)cV[(32 * j + 8 * lg + e) * LDK + 16 * d + lr];
    return C::make(x);
  };
  using SAcc = f32x4[QT][2];
  using KFr = Frag[KS][2];
  using VFr = VFrag[DT];
  // K-hat fragments of block j: key kv = 8*(r/4) + 4*h + r%4 in A-row r of half h
  auto load_k = [&](const S* __restrict__ cK, int j, KFr& kf) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int h = 0; h < 2; ++h) kf[s][h] = C::lds(&cK[(32 * j + 16 * h + lr) * LDK + 32 * s + 8 * lg]);
  };
  // V^T fragments of block j: A = V^T rows 16d.., k-slot e <-> key 32j + 8lg + e (the P^T order)
  auto load_v = [&](const VS* __restrict__ cV, int j, VFr& vf) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      if constexpr (TRV)
        vf[d] = VC::tr(cV + (32 * j + vr0) * LDK + 16 * d + 4 * (lr & 3),
                      cV + (32 * j + vr1) * LDK + 16 * d + 4 * (lr & 3));
      else if constexpr (VROW)
        vf[d] = vrow_frag(cV, j, d);
      else
        vf[d] = C::lds(&cV[(16 * d + lr) * LDV + vswz(16 * d + lr, 32 * j + 8 * lg)]);
    }
  };
  // S^T = K-hat Q-hat^T for 32 keys (each K-hat fragment feeds QT MFMAs)
  auto logits = [&](const KFr& kf, SAcc& sa) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < QT; ++t) sa[t][0] = sa[t][1] = f32x4{-mb[t], -mb[t], -mb[t], -mb[t]};
    if constexpr (!FS) {   // (the pipelined chunk runs without fp16 operands)
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int t = 0; t < QT; ++t) sa[t][h] = C::mma(kf[s][h], qf[t][s], sa[t][h]);
    }
  };
  // Online softmax of one block; the lane holds keys 8lg + (0..7) of the
  // block for its query row.  MASKED: keys e >= lim get probability 0.
  // The running max only has to bound the exponent: O and the row sum are
  // rescaled (group max, times 2^(m_old - m_new)) only when some lane's own
  // max exceeds m_run + slack.  The block's values arrive as logits minus
  // m_run (accumulators seeded with -mb, all in log2 units through the
  // pre-scaled K-hat), so the test is against m_thr = slack (-inf before
  // the first block) and P is exp2 of the values themselves.
  //
  // The common case has no branch: soft() computes P with the current
  // running max and reports whether any row crossed its threshold; only then
  // does fixup() rescale and recompute the block (rare after an item's first
  // block).  Straight-line code lets the scheduler interleave these VALU
  // instructions with the MFMAs of the neighbouring blocks.
  auto block_vals = [&](auto maskc, const SAcc& sa, int t, int lim, float (&sv)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) sv[4 * h + i] = sa[t][h][i];
    if constexpr (decltype(maskc)::value) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sv[e] = e < lim ? sv[e] : -INFINITY;
    }
  };
  auto max8 = [](const float (&sv)[8]) __attribute__((always_inline)) {
    return fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])), fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
  };
  // sv: logits minus the running max (the seeded accumulators)
  auto probs = [&](const float (&sv)[8], int t, VFrag& pft) __attribute__((always_inline)) {
    float pv8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pv8[e] = fast_exp2(sv[e]);
      l_run[t] += pv8[e];
    }
    if constexpr (FS)
      pft.v = to_f16x8(pv8);
    else
      pft = C::make(pv8);
  };
  auto soft = [&](auto maskc, const SAcc& sa, int lim, VFrag (&pf)[QT], float (&lkeep)[QT]) __attribute__((always_inline)) {
    bool need = false;
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      float sv[8];
      block_vals(maskc, sa, t, lim, sv);
      need |= __any(max8(sv) > m_thr[t]);
      lkeep[t] = l_run[t];
      probs(sv, t, pf[t]);
    }
    return need;
  };
  // The new base also applies to a block whose logits are already issued
  // (pend): its accumulators are shifted by the change.
  auto fixup = [&](auto maskc, const SAcc& sa, int lim, VFrag (&pf)[QT], const float (&lkeep)[QT],
                   SAcc* pend) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      float sv[8];
      block_vals(maskc, sa, t, lim, sv);
      const float mx = group4_max(max8(sv)) + mb[t];
      const float mnew = fmaxf(m_run[t], mx);
      const float alpha = fast_exp2(m_run[t] - mnew);
      l_run[t] = lkeep[t] * alpha;
#pragma unroll
      for (int d = 0; d < DT; ++d) oacc[t][d] *= alpha;
      m_run[t] = mnew;
      const float mbn = mnew == -INFINITY ? mb[t] : mnew;
      const float shift = mb[t] - mbn;
      mb[t] = mbn;
      m_thr[t] = kRescaleSlack;
#pragma unroll
      for (int e = 0; e < 8; ++e) sv[e] += shift;
      probs(sv, t, pf[t]);
      if (pend) {
#pragma unroll
        for (int h = 0; h < 2; ++h) (*pend)[t][h] += shift;
      }
    }
  };
  auto softmax = [&](auto maskc, const SAcc& sa, int lim, VFrag (&pf)[QT], SAcc* pend) __attribute__((always_inline)) {
    float lkeep[QT];
    if (soft(maskc, sa, lim, pf, lkeep)) fixup(maskc, sa, lim, pf, lkeep, pend);
  };
  // O^T += V^T P^T (each V^T fragment feeds QT MFMAs)
  auto out_mma = [&](const VFr& vf, const VFrag (&pf)[QT]) __attribute__((always_inline)) {
#pragma unroll
    for (int d = 0; d < DT; ++d)
#pragma unroll
      for (int t = 0; t < QT; ++t) oacc[t][d] = VC::mma(vf[d], pf[t], oacc[t][d]);
  };
  // One KV chunk of nb blocks; the block holding key N-1 is the last one of
  // the chunk that starts at kvb (the ragged chunk is processed first).
  auto chunk = [&](const S* __restrict__ cK, const VS* __restrict__ cV, int kvb, bool active, auto&& mem) __attribute__((always_inline)) {
    const int nkeys = min(KC, N - kvb);
    // a wave with no query row below N runs one block (its results are never
    // stored) so that every wave reaches mem() on the same straight-line path
    const int nb = active ? (nkeys + 31) >> 5 : 1;
    SAcc s0, s1;
    KFr ka, kb;
    VFr vf;
    VFrag pf[QT];
    load_k(cK, 0, ka);
    logits(ka, s0);
    load_k(cK, min(1, nb - 1), kb);
    // The chunk's prefetch loads issue here, under the first block's
    // products, rather than in a burst before the barrier.
    __builtin_amdgcn_sched_barrier(0);
    mem();
    __builtin_amdgcn_sched_barrier(0);
    // Step j: the logits of block j+1 (its K-hat is already in registers) go
    // to the MFMA pipe first and run under block j's softmax; block j+2's
    // K-hat (into the registers block j's K-hat has left) and block j's V^T
    // load meanwhile.  Two blocks per trip, so the logits and K-hat registers
    // alternate without copies; past the last block the K-hat load re-reads
    // the last block.
    auto step = [&](int j, const SAcc& cur, SAcc& nxt, const KFr& kn, KFr& kfree) __attribute__((always_inline)) {
      logits(kn, nxt);
      load_k(cK, min(j + 2, nb - 1), kfree);
      load_v(cV, j, vf);
      softmax(std::false_type{}, cur, 8, pf, &nxt);
      out_mma(vf, pf);
    };
    auto last = [&](int j, const SAcc& cur) __attribute__((always_inline)) {
      load_v(cV, j, vf);
      if (nkeys & 31)
        softmax(std::true_type{}, cur, N - (kvb + 32 * j + 8 * lg), pf, nullptr);
      else
        softmax(std::false_type{}, cur, 8, pf, nullptr);
      out_mma(vf, pf);
    };
    int j = 0;
    for (; j + 2 < nb; j += 2) {
      step(j, s0, s1, kb, ka);
      step(j + 1, s1, s0, ka, kb);
    }
    if (j + 1 < nb) {
      logits(kb, s1);
      load_v(cV, j, vf);
      softmax(std::false_type{}, s0, 8, pf, &s1);
      out_mma(vf, pf);
      last(j + 1, s1);
    } else {
      last(j, s0);
    }
  };

  // Without the LDS table (D = 128 or long planes), or with 32-bit I/O (twice
  // the prefetch registers), the registers of the pipeline are not free: the
  // same work block by block.
  constexpr bool kPipe = kTabLds && sizeof(IO) == 2 && !FS;
  // One KV chunk for all QT subtiles of the wave.  Subtiles past the last
  // query row hold zero rows and are computed anyway: every wave of a
  // workgroup then runs the same instruction stream with no per-subtile
  // guards, and for the 16-row-ragged N of ViT planes the extra work lands on
  // SIMDs that would otherwise wait at the next barrier.
  // One 32-key block for all QT subtiles of the wave, in two halves so that a
  // chunk can software-pipeline them: blk_logits issues the S^T products of a
  // block, blk_out its online softmax and O^T += V^T P^T.  Subtiles past the
  // last query row hold zero rows and are computed anyway: every wave of a
  // workgroup then runs the same instruction stream with no per-subtile
  // guards.  MASKED: the block holding key N-1 (keys >= N get probability 0).
  auto blk_logits = [&](const S* __restrict__ cK, int j, SAcc& sacc) __attribute__((always_inline)) {
    // ---- S^T = K-hat Q-hat^T for 32 keys (each K-hat fragment feeds QT MFMAs) ----
#pragma unroll
    for (int t = 0; t < QT; ++t) sacc[t][0] = sacc[t][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int off = (32 * j + 16 * h + lr) * LDK + 32 * s + 8 * lg;
        const LFrag a = LC::lds(reinterpret_cast<const typename LC::S*>(&cK[off]));
#pragma unroll
        for (int t = 0; t < QT; ++t) sacc[t][h] = LC::mma(a, qf[t][s], sacc[t][h]);
      }
    }
  };
  auto blk_out = [&](auto maskc, const VS* __restrict__ cV, int kvb, int j, const SAcc& sacc)
      __attribute__((always_inline)) {
    constexpr bool MASKED = decltype(maskc)::value;
    // fp16 logits (vector access): the first kVPre V^T fragments are read before
    // its softmax, so that their LDS latency passes under it (the compiler
    // otherwise issues each read next to its product and waits for it there;
    // 4 fit the register budget: HiRes forward -6 us)
    constexpr int kVPre = (TRV && FS && VEC) ? 4 : 0;
    VFrag vpre[kVPre > 0 ? kVPre : 1];
    if constexpr (kVPre > 0) {
#pragma unroll
      for (int d = 0; d < kVPre; ++d)
        vpre[d] = VC::tr(cV + (32 * j + vr0) * LDK + 16 * d + 4 * (lr & 3), cV + (32 * j + vr1) * LDK + 16 * d + 4 * (lr & 3));
      __builtin_amdgcn_sched_barrier(0);
    }
    // ---- online softmax; lane holds keys kvb + 32j + 8lg + (0..7) of its row ----
    const int lim = N - (kvb + 32 * j + 8 * lg);   // keys e < lim are valid (MASKED only)
    VFrag pf[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      float sv[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[4 * h + i] = sacc[t][h][i];
      if constexpr (MASKED) {
#pragma unroll
        for (int e = 0; e < 8; ++e) sv[e] = e < lim ? sv[e] : -INFINITY;
      }
      // The running max only has to bound the exponent: rescale (group max,
      // O and row sum times 2^(m_old - m_new)) only when some lane's own max
      // exceeds m_thr = m_run + slack (log2 units).  FS: the logits are
      // fsc * sv (fsc = 1 except in a rescaled pass), folded into the max
      // and into the exponent's subtraction.
      float ml = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                       fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
      if constexpr (FS) ml *= fsc;
      if (__any(ml > m_thr[t])) {
        const float mx = group4_max(ml);
        const float mnew = fmaxf(m_run[t], mx);
        const float alpha = fast_exp2(m_run[t] - mnew);
        l_run[t] *= alpha;
#pragma unroll
        for (int d = 0; d < DT; ++d) oacc[t][d] *= alpha;
        m_run[t] = mnew;
        m_thr[t] = mnew + kRescaleSlack;
      }
      float pv8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv8[e] = fast_exp2(FS ? __builtin_fmaf(sv[e], fsc, -m_run[t]) : sv[e] - m_run[t]);
        l_run[t] += pv8[e];
      }
      if constexpr (FS)
        pf[t].v = to_f16x8(pv8);
      else
        pf[t] = C::make(pv8);
    }
    // ---- O^T += V^T P^T (each V^T fragment feeds QT MFMAs) ----
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      // A = V^T rows 16d.., k-slot e <-> key 32j + 8lg + e (the P^T order)
      VFrag a;
      if constexpr (TRV) {
        if (d < kVPre)
          a = vpre[d < kVPre ? d : 0];
        else
          a = VC::tr(cV + (32 * j + vr0) * LDK + 16 * d + 4 * (lr & 3), cV + (32 * j + vr1) * LDK + 16 * d + 4 * (lr & 3));
      } else if constexpr (VROW) {
        a = vrow_frag(cV, j, d);
      } else {
        a = C::lds(&cV[(16 * d + lr) * LDV + vswz(16 * d + lr, 32 * j + 8 * lg)]);
      }
#pragma unroll
      for (int t = 0; t < QT; ++t) oacc[t][d] = VC::mma(a, pf[t], oacc[t][d]);
    }
  };
  // One KV chunk of nb blocks (the last one ragged when N - kvb < KC and not
  // a multiple of 32).  With one subtile per wave, or two at D >= 128 with
  // 16-bit operands and vector access, the logits of block j+1 are issued
  // before the softmax of block j, so that those MFMAs run while the VALU
  // computes block j's probabilities; two blocks per trip alternate the two
  // logit accumulators without copies.
  // MASKC: the chunk may hold keys >= N (an item's first chunk, the ragged
  // one); the other chunks of an item are full.
  auto chunk_serial = [&](auto maskc, const S* __restrict__ cK, const VS* __restrict__ cV, int kvb) __attribute__((always_inline)) {
    const int nkeys = min(KC, N - kvb);
    if constexpr (sizeof(S) == 2 && (QT == 1 || (VEC && D >= 128))) {
      // every block of a chunk goes through the same softmax (with MASKC the
      // masked one, with a key limit past the block for full ones): one
      // inlined copy per call site keeps the pipelined loop within the
      // register budget
      const int nb = (nkeys + 31) >> 5;
      SAcc sA, sB;
      blk_logits(cK, 0, sA);
      int j = 0;
      for (; j + 1 < nb; j += 2) {
        blk_logits(cK, j + 1, sB);
        blk_out(maskc, cV, kvb, j, sA);
        if (j + 2 < nb) blk_logits(cK, j + 2, sA);
        blk_out(maskc, cV, kvb, j + 1, sB);
      }
      if (j < nb) blk_out(maskc, cV, kvb, j, sA);   // odd block count: last logits in sA
    } else {
      // two subtiles per wave at D <= 64 or with element-wise access, or fp32
      // compute (split operands): two blocks' logits do not fit beside their
      // accumulators, so block by block
      const int nfull = nkeys / 32;
      SAcc sA;
      for (int j = 0; j < nfull; ++j) {
        blk_logits(cK, j, sA);
        blk_out(std::false_type{}, cV, kvb, j, sA);
      }
      if (nkeys % 32) {
        blk_logits(cK, nfull, sA);
        blk_out(std::true_type{}, cV, kvb, nfull, sA);
      }
    }
  };

  int it = 0;
  int item = item_of(0);
  if (item < 0) return;
  KvRs kvr = kv_rs(item);
  prefetch_kv(item, kvr, 0);
  prefetch_q(item);
  if constexpr (kTabLds) {
    // rows 0 .. N-1+shift of the packed table (TCH 16-byte chunks each), swizzled
    const f32x4* src = reinterpret_cast<const f32x4*>(p.rope);
    for (int i = tid; i < (N + shift) * TCH; i += NT) {
      const int r = i / TCH, c = i - r * TCH;
      *reinterpret_cast<f32x4*>(&sTab[(r * TCH + (c ^ (r & (TCH - 1)))) * 4]) = src[i];
    }
    lds_barrier();
  }
  int g = 0;   // chunks consumed so far: LDS slot g & 1

  // VEC, 16-bit I/O: an item's O rows and LSE are stored during the next
  // item, right after that item's first KV chunk has arrived.  Stores and
  // loads share one in-order wait counter, so O stores issued at the end of
  // an item would make the next item's waits for its prefetched Q and KV rows
  // also wait for the stores to complete.  Deferred, the stores are older
  // than every load waited on later and have a whole chunk of compute to
  // drain.  The stores are unconditional: rows >= N fall outside the
  // descriptor range and are dropped, LSE lanes lg != 0 write past their
  // range, and before the first item the ranges are empty.
  // (Not with Q rows loaded at the item start: those loads wait for the
  // stores either way, and the deferred store registers would not fit.)
  constexpr bool kDefer = VEC && sizeof(IO) == 2 && kQpf;
  u32x2 ost[kDefer ? QT : 1][DT];
  // RES: O's rounding residual bf16(O - bf16(O)) goes to p.o_res (contiguous
  // [B, H, N, D]) next to O, for the backward's delta; stored only when the
  // caller gave the buffer (a uniform test)
  constexpr bool RES = FS && std::is_same<IO, bf16>::value;
  u32x2 ostr[kDefer && RES ? QT : 1][DT];
  auto res4 = [](const float (&o4)[4], const IO (&h4)[4], float (&r4)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 4; ++r) r4[r] = o4[r] - (float)h4[r];
  };
  float olse[QT];
  int orow[QT];
  int oplane = -1;
  auto flush_o = [&]() __attribute__((always_inline)) {
    if constexpr (kDefer) {
      const bool have = oplane >= 0;
      const int pl = have ? oplane : 0;
      const auto rO = make_rsrc(plane_base(p.o, p.so, pl),
                                have ? (unsigned)(((int64_t)(N - 1) * p.so[2] + D) * ES) : 0u);
      const auto rL = make_rsrc(p.lse + (int64_t)pl * N, have ? (unsigned)N * 4u : 0u);
      const bool res = RES && p.o_res != nullptr;
      const auto rR = make_rsrc(static_cast<IO*>(res ? p.o_res : p.o) + (int64_t)pl * N * D,
                                have && res ? (unsigned)N * D * ES : 0u);
      // Lane groups lg and lg^1 trade halves so that each lane writes 8
      // consecutive channels (16 bytes) per pair of 16-channel slices
      // (d0, d1): v_permlane16_swap(a, b) gives even lane groups {a, a of
      // lg+1} and odd ones {b of lg-1, b}.  Even lg then holds channels
      // 16d0 + 4lg .. +7, odd lg channels 16d1 + 4(lg-1) .. +7.
      const int cbase = 4 * (lg & 2);
#pragma unroll
      for (int t = 0; t < QT; ++t) {
#pragma unroll
        for (int d0 = 0; d0 < DT; d0 += 2) {
          u32x4 w;
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            const auto r = __builtin_amdgcn_permlane16_swap(ost[t][d0][k], ost[t][d0 + 1][k], false, false);
            w[k] = r[0];
            w[2 + k] = r[1];
          }
          const int ch = 16 * (d0 + (lg & 1)) + cbase;
          buf_store16(w, rO, (unsigned)((orow[t] * (int)p.so[2] + ch) * (int)ES), 0u);
          if constexpr (RES) {
            u32x4 wr;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const auto r = __builtin_amdgcn_permlane16_swap(ostr[t][d0][k], ostr[t][d0 + 1][k], false, false);
              wr[k] = r[0];
              wr[2 + k] = r[1];
            }
            // empty range (stores dropped) when there is no residual buffer
            buf_store16(wr, rR, (unsigned)((orow[t] * D + ch) * (int)ES), 0u);
          }
        }
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(olse[t]), rL,
                                              (unsigned)(lg == 0 ? orow[t] : N) * 4u, 0u, 0);
      }
    }
  };
  while (item >= 0) {
    const int plane = item / p.n_blk, qb = item - plane * p.n_blk;
    const int nxt = item_of(it + 1);
    if constexpr (XR) {
      // the designated item of a plane cycles through the q blocks with the
      // plane's launch iteration, so the extra rows spread over workgroups
      xi = p.x_rows != 0 && qb == (plane / max(1, p.n_wg / p.n_blk)) % p.n_blk;
    }
    if constexpr (kQdesc) load_q(plane, qb);
    commit_q(plane, qb);
    int nt = 0;   // active subtiles of this wave: a prefix t < nt (wave-uniform)
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      nt += (qb * NW * QT + t * NW + wave) * 16 < N;
      m_run[t] = -INFINITY;
      m_thr[t] = -INFINITY;
      mb[t] = 0.f;
      l_run[t] = 0.f;
#pragma unroll
      for (int d = 0; d < DT; ++d) oacc[t][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // One KV chunk: stage it into LDS, start the next chunk (or the next
    // item's first chunk) with one call on a uniformly selected target, and --
    // after the first chunk is staged -- the next item's Q rows (the last item
    // re-reads its own).  Unconditional loads with no merge copies let every
    // wait cover exactly the load it needs.
    auto chunk_step = [&](auto firstc, int c) __attribute__((always_inline)) {
      constexpr bool FIRST = decltype(firstc)::value;
      const int slot = g & 1;
      commit_kv(slot, chunk_start(c));
      if constexpr (FS) {
        // After the item's last K-hat chunk is converted: the operand ranges
        // of this pass over the workgroup (each wave's, through LDS, read
        // between this barrier and the next; the next pass writes after
        // both).  If Q-hat or K-hat reached 2^12, the item is computed again
        // with scaled operands, and the prefetch below loads its first chunk
        // once more.
        if (c == nch - 1) {
          {
            const unsigned rq = wave_max_bits(amax_q), rk = wave_max_bits(amax_k), rv = wave_max_bits(amax_vf);
            if (lane == 0) sRange[wave] = u32x4{rq, rk, rv, 0u};
          }
          lds_barrier();
          unsigned rq = 0, rk = 0, rv = 0;
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const u32x4 r = sRange[w];
            rq = max(rq, r[0]);
            rk = max(rk, r[1]);
            rv = max(rv, r[2]);
          }
          eq = __builtin_amdgcn_readfirstlane(rq) >> 23;
          ek = __builtin_amdgcn_readfirstlane(rk) >> 23;
          ev = __builtin_amdgcn_readfirstlane(rv) >> 23;
          // (ev == 0: V is zero, nothing to resolve)
          redo = !rescaled && (eq >= kF16ExpLimit || ek >= kF16ExpLimit || ev >= kF16ExpLimit ||
                               (ev != 0u && ev < kF16ExpLow));
        }
      }
      if constexpr (FIRST && kPipe) flush_o();
      auto mem = [&]() __attribute__((always_inline)) {
        if constexpr (FIRST) {
          if constexpr (!kPipe) flush_o();
          // the next item's Q rows before the next KV chunk: Q is waited for
          // first, at the next item's start, so at least one KV load is younger
          // and stays in flight across that wait (also when nch == 1)
          prefetch_q(nxt >= 0 ? nxt : item);
        }
        const bool last = c + 1 == nch;
        const int tgt = last && !redo ? (nxt >= 0 ? nxt : item) : item;
        if (last) kvr = kv_rs(tgt);
        prefetch_kv(tgt, kvr, last ? 0 : c + 1);
      };
      // The O stores and the Q/KV prefetch of a chunk switch (~96 KB per
      // workgroup at 64 channels) pass through the CU's vector memory path
      // in over a thousand cycles, and a wave stalls at issue while that path
      // is full.  Issued before the barrier, the loads hold every wave there;
      // the pipelined chunk issues them after its first products instead, so
      // they drain while the SIMDs compute.  (The stores stay before the
      // barrier: issued under the products they stalled the first block.)
      if constexpr (kPipe) {
        lds_barrier();
        chunk(sK[slot], sVt[slot], chunk_start(c), nt > 0, mem);
      } else {
        mem();
        lds_barrier();
        // (chunk 0 starts at the last chunk's keys: only it can hold keys >= N)
        if (nt > 0) chunk_serial(firstc, sK[slot], sVt[slot], chunk_start(c));
        if constexpr (XR) {
          if (xi) xrow_chunk(sK[slot], sVt[slot], chunk_start(c), c == 0);
        }
      }
      ++g;
    };
    chunk_step(std::true_type{}, 0);
    for (int c = 1; c < nch; ++c) chunk_step(std::false_type{}, c);

    if constexpr (FS) {
      // a rescaled second pass (its first chunk is already on the way; no
      // Q prefetch or deferred store exists with these operands); no store
      amax_q = amax_k = amax_vf = 0.f;
      if constexpr (XR) ++npass;
      if (redo) {
        redo = false;
        rescaled = true;
        fq = f16_fit(eq);
        fk = f16_fit(ek);
        fsc = 1.f / (fq * fk);
        fv = ev != 0u ? f16_fit(ev) : 1.f;
        continue;
      }
      ifv = 1.f / fv;
      rescaled = false;
      fq = fk = fsc = fv = 1.f;
    }
    if constexpr (XR) {
      if (xi) {
        // merge the waves' partial states of the last row: M = max m_w,
        // L = sum l_w 2^(m_w - M), O = sum o_w 2^(m_w - M) / L
        lds_barrier();
        if (wave == 0) {
          const int ln = opaque(lane);
          float M = -INFINITY;
#pragma unroll
          for (int w = 0; w < NW; ++w) M = fmaxf(M, sXml[w][0]);
          float L = 0.f, o[XO] = {};
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const float a = fast_exp2(sXml[w][0] - M);
            L = __builtin_fmaf(sXml[w][1], a, L);
#pragma unroll
            for (int i = 0; i < XO; ++i) o[i] = __builtin_fmaf(sXo[w][XO * ln + i], a, o[i]);
          }
          const float inv = ifv / L;
          IO* orow_p = const_cast<IO*>(plane_base(p.o, p.so, plane)) + (N - 1) * p.so[2] + XO * ln;
          typedef IO iox __attribute__((ext_vector_type(XO)));
          iox h, rr;
#pragma unroll
          for (int i = 0; i < XO; ++i) {
            o[i] *= inv;
            h[i] = (IO)o[i];
            rr[i] = (IO)(o[i] - (float)h[i]);
          }
          *reinterpret_cast<iox*>(orow_p) = h;
          if constexpr (RES) {
            if (p.o_res) *reinterpret_cast<iox*>(static_cast<IO*>(p.o_res) + ((int64_t)plane * N + N - 1) * D + XO * ln) = rr;
          }
          if (ln == 0) p.lse[(int64_t)plane * N + N - 1] = (M + fast_log2(L)) * kLn2;
        }
      }
    }

    // ---- epilogue: lane holds O[row][16d + 4lg + (0..3)] ----
    if constexpr (kDefer) {
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const float l = group4_sum(l_run[t]);
        const float inv = __builtin_amdgcn_rcpf(l);
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          typedef IO io4 __attribute__((ext_vector_type(4)));
          io4 a;
          float o4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            o4[r] = oacc[t][d][r] * inv;
            a[r] = (IO)o4[r];
          }
          __builtin_memcpy(&ost[t][d], &a, 8);
          if constexpr (RES) {
            io4 b;
#pragma unroll
            for (int r = 0; r < 4; ++r) b[r] = (IO)(o4[r] - (float)a[r]);
            __builtin_memcpy(&ostr[t][d], &b, 8);
          }
        }
        olse[t] = (m_run[t] + fast_log2(l)) * kLn2;
        orow[t] = (qb * NW * QT + t * NW + wave) * 16 + lr;
      }
      oplane = plane;
    } else if constexpr (VEC) {
      // Unconditional descriptor stores: rows >= N (every row of an inactive
      // subtile included) fall outside the plane's range and are dropped, and
      // the LSE of lanes lg != 0 goes to an offset past its range.  With no
      // branch around them the wait counter keeps counting these stores
      // exactly, so the next item's waits for its prefetched rows do not also
      // wait for the stores to complete.
      const auto rO = rsrc(p.o, p.so, plane);
      const auto rL = make_rsrc(p.lse + (int64_t)plane * N, (unsigned)N * 4u);
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const float l = group4_sum(l_run[t]);
        const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
        const float inv = __builtin_amdgcn_rcpf(l) * ifv;
        if constexpr (sizeof(IO) == 2 && DT % 2 == 0) {
          // 16-byte stores, half as many store instructions: lane groups lg
          // and lg^1 trade halves (v_permlane16_swap, as in flush_o).  Every
          // workgroup ends its items at about the same time, and the 8-byte
          // stores of O and its residual (32 per wave) held the waves at
          // issue: HiRes forward -14 us.  (Rows >= N and, without a residual
          // buffer, the residual stores fall outside their ranges.)
          const bool res = RES && p.o_res != nullptr;
          const auto rR = make_rsrc(static_cast<IO*>(RES && p.o_res ? p.o_res : p.o) + (int64_t)plane * N * D,
                                    res ? (unsigned)N * D * ES : 0u);
          const int cbase = 4 * (lg & 2);
#pragma unroll
          for (int d0 = 0; d0 < DT; d0 += 2) {
            u32x2 wo[2], wr[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              typedef IO io4 __attribute__((ext_vector_type(4)));
              io4 a, b;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float o = oacc[t][d0 + h][r] * inv;
                a[r] = (IO)o;
                b[r] = (IO)(o - (float)a[r]);
              }
              __builtin_memcpy(&wo[h], &a, 8);
              __builtin_memcpy(&wr[h], &b, 8);
            }
            u32x4 w, x;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
              const auto r1 = __builtin_amdgcn_permlane16_swap(wo[0][k], wo[1][k], false, false);
              w[k] = r1[0];
              w[2 + k] = r1[1];
              const auto r2 = __builtin_amdgcn_permlane16_swap(wr[0][k], wr[1][k], false, false);
              x[k] = r2[0];
              x[2 + k] = r2[1];
            }
            const int ch = 16 * (d0 + (lg & 1)) + cbase;
            buf_store16(w, rO, (unsigned)((row * (int)p.so[2] + ch) * (int)ES), 0u);
            if constexpr (RES) buf_store16(x, rR, (unsigned)((row * D + ch) * (int)ES), 0u);
          }
        } else {
#pragma unroll
        for (int d = 0; d < DT; ++d) {
          float o4[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) o4[r] = oacc[t][d][r] * inv;
          buf_store4<IO>(rO, (unsigned)((row * (int)p.so[2] + 16 * d + 4 * lg) * (int)ES), 0u, o4);
          if constexpr (RES) {
            if (p.o_res) {
              IO h4[4];
              float r4[4];
#pragma unroll
              for (int r = 0; r < 4; ++r) h4[r] = (IO)o4[r];
              res4(o4, h4, r4);
              const auto rR = make_rsrc(static_cast<IO*>(p.o_res) + (int64_t)plane * N * D, (unsigned)N * D * ES);
              buf_store4<IO>(rR, (unsigned)((row * D + 16 * d + 4 * lg) * (int)ES), 0u, r4);
            }
          }
        }
        }
        const float lse = (m_run[t] + fast_log2(l)) * kLn2;
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(lse), rL, (unsigned)(lg == 0 ? row : N) * 4u, 0u, 0);
      }
    } else {
      IO* __restrict__ O = const_cast<IO*>(plane_base(p.o, p.so, plane));
#pragma unroll
      for (int t = 0; t < QT; ++t) {
        const float l = group4_sum(l_run[t]);
        const int row = (qb * NW * QT + t * NW + wave) * 16 + lr;
        if (t < nt && row < N) {
          const float inv = __builtin_amdgcn_rcpf(l) * ifv;
#pragma unroll
          for (int d = 0; d < DT; ++d) {
            float o4[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) o4[r] = oacc[t][d][r] * inv;
            store4(O + row * p.so[2] + (16 * d + 4 * lg) * p.so[3], p.so[3], vec_o, o4);
            if constexpr (RES) {
              if (p.o_res) {
                IO h4[4];
                float r4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) h4[r] = (IO)o4[r];
                res4(o4, h4, r4);
                IO* R = static_cast<IO*>(p.o_res) + ((int64_t)plane * N + row) * D + 16 * d + 4 * lg;
                store4(R, 1, true, r4);
              }
            }
          }
          if (lg == 0) p.lse[(int64_t)plane * N + row] = (m_run[t] + fast_log2(l)) * kLn2;
        }
      }
    }
    item = nxt;
    ++it;
  }
  flush_o();
}

// ---------------------------------------------------------------------------
// Tile table for the forward pass: (NW, QT, KC) per head_dim.  One work item
// covers NW*QT*16 query rows of a plane; workgroups are persistent.
// ---------------------------------------------------------------------------
// TABROWS: rows of the packed RoPE table an LDS-resident copy can hold
// (N + 1 - has_cls <= TABROWS; i.e. planes up to 256 tokens).
template <int D> struct FwdShape;
template <> struct FwdShape<32> { static constexpr int NW = 8, QT = 2, KC = 128, TABROWS = 257; };
template <> struct FwdShape<64> { static constexpr int NW = 8, QT = 2, KC = 128, TABROWS = 257; };
template <> struct FwdShape<128> { static constexpr int NW = 8, QT = 1, KC = 64, TABROWS = 0; };
// D = 256: one wave per SIMD (4-wave workgroups), so each wave may hold up to
// 512 registers (VGPRs plus AGPRs): the O accumulators alone are 64 per wave.
template <> struct FwdShape<256> { static constexpr int NW = 4, QT = 1, KC = 32, TABROWS = 0; };

// Query subtiles per wave at D = 128: two with 16-bit tensors and 16-bit
// compute, so that every staged K-hat chunk (rotated and converted once per
// item) serves twice the queries; their Q rows
// then load at the item start (no prefetch).  32-bit tensors or compute need
// those registers for staging.
template <int D, int CT, bool IO16> constexpr int fwd_qt() {
  return IO16 && CT != DT_F32 && D == 128 ? 2 : FwdShape<D>::QT;
}
template <int D> static int fwd_rows_of(int io, int ct) {
  const bool two = io != DT_F32 && ct != DT_F32;
  return FwdShape<D>::NW * (two ? fwd_qt<D, DT_BF16, true>() : FwdShape<D>::QT) * 16;
}
int fwd_block_rows(int D, int io, int ct) {
  return D == 32 ? fwd_rows_of<32>(io, ct) : D == 64 ? fwd_rows_of<64>(io, ct)
         : D == 128 ? fwd_rows_of<128>(io, ct) : fwd_rows_of<256>(io, ct);
}
int fwd_threads(int D) {
  return 64 * (D == 32    ? FwdShape<32>::NW
               : D == 64  ? FwdShape<64>::NW
               : D == 128 ? FwdShape<128>::NW
                          : FwdShape<256>::NW);
}

template <typename IO, int CT, int D>
static hipError_t fwd_launch(const FwdParams& p0, hipStream_t st) {
  using SH = FwdShape<D>;
  FwdParams p = p0;
  // fp32 compute keeps 4-byte tiles in LDS: no room for the table copy there
  constexpr int TR = CT == DT_F32 ? 0 : SH::TABROWS;
  // fp16 logit operands for bf16 compute at head_dim >= 128 (the backward's
  // split kernels use the same rule, so both passes see the same S)
  constexpr bool FS = f16_logits(CT, D);
  constexpr int QT = fwd_qt<D, CT, sizeof(IO) == 2>();
  const bool tab = TR > 0 && p.N + 1 - p.has_cls <= TR;
  const bool vec = p.vec_q && p.vec_k && p.vec_v && p.vec_o;
  auto kern = tab ? (vec ? fwd_kernel<IO, CT, D, SH::NW, QT, SH::KC, TR, true, FS>
                         : fwd_kernel<IO, CT, D, SH::NW, QT, SH::KC, TR, false, FS>)
                  : (vec ? fwd_kernel<IO, CT, D, SH::NW, QT, SH::KC, 0, true, FS>
                         : fwd_kernel<IO, CT, D, SH::NW, QT, SH::KC, 0, false, FS>);
  const int grid = persistent_grid(reinterpret_cast<const void*>(kern), SH::NW * 64, p.n_items);
  if (grid <= 0) return hipErrorInvalidConfiguration;
  p.n_wg = grid;
  hipLaunchKernelGGL(kern, dim3(grid), dim3(SH::NW * 64), 0, st, p);
  return hipGetLastError();
}

template <typename IO, int CT>
static hipError_t fwd_shape(const FwdParams& p, int D, hipStream_t st) {
  switch (D) {
    case 32: return fwd_launch<IO, CT, 32>(p, st);
    case 64: return fwd_launch<IO, CT, 64>(p, st);
    case 128: return fwd_launch<IO, CT, 128>(p, st);
    default: return fwd_launch<IO, CT, 256>(p, st);
  }
}

template <typename IO>
static hipError_t fwd_ct(const FwdParams& p, int ct, int D, hipStream_t st) {
  switch (ct) {
    case DT_BF16: return fwd_shape<IO, DT_BF16>(p, D, st);
    case DT_F16: return fwd_shape<IO, DT_F16>(p, D, st);
    default: return fwd_shape<IO, DT_F32>(p, D, st);
  }
}

bool fwd_folds_tail(int io, int ct, int D, bool vec) {
  // the XR instantiations: 16-bit I/O, fp16 logits, KC = 8 NW (D = 128, 256)
  return io != DT_F32 && f16_logits(ct, D) && vec && (D == 128 || D == 256);
}

hipError_t launch_fwd(const FwdParams& p, int io, int ct, int D, hipStream_t st) {
  switch (io) {
    case DT_BF16: return fwd_ct<bf16>(p, ct, D, st);
    case DT_F16: return fwd_ct<f16>(p, ct, D, st);
    default: return fwd_ct<float>(p, ct, D, st);
  }
}

}  // namespace farope
