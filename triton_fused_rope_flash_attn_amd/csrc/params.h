// Kernel argument blocks (passed by value) and the launcher declarations that
// connect the C-ABI layer (api.hip) to the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace farope {

// One (b, h) plane of a [B, H, N, D] tensor starts at b*s[0] + h*s[1]
// elements; row n, channel d at n*s[2] + d*s[3].
struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  void* o_res;         // optional contiguous [B, H, N, D]: bf16(O - bf16(O)) (see o_residual)
  float* lse;          // [B*H, N] fp32, natural-log log-sum-exp of the logits
  int64_t sq[4], sk[4], sv[4], so[4];
  const float* rope;   // packed (cos, sin) table [(n_pos + 1), D/2, 2]
  int B, H, N, has_cls;
  float scale_log2;    // softmax_scale * log2(e)
  int vec_q, vec_k, vec_v, vec_o;
  int n_blk;           // q blocks per plane
  int n_items;         // planes * n_blk work items
  int n_wg;            // workgroups of the launch (set by the launcher)
  int x_rows;          // 1: the block kernel also computes row N - 1 (fwd_folds_tail)
};

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* o_res;   // optional contiguous [B, H, N, D]: O's rounding residual, added to O for delta
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  const float* lse;    // [B*H, N]
  float* delta;        // [B*H, N]: rowsum(dO * O)
  int64_t sq[4], sk[4], sv[4], so[4], sdo[4], sdq[4], sdk[4], sdv[4];
  const float* rope;
  int B, H, N, has_cls;
  float scale;         // softmax_scale
  float scale_log2;    // softmax_scale * log2(e)
  int vec_q, vec_k, vec_v, vec_o, vec_do, vec_dq, vec_dk, vec_dv;
  int n_blk;           // q blocks (dq kernel) or kv blocks (dk/dv kernel) per plane
  int n_wg;            // workgroups of the launch (set by the launcher)
  int x_rows;          // 1: the dQ block kernel also computes row N - 1 (bwd_folds_tail)
  float* xk_ws;        // non-null: the dQ kernel's tiles write their partial dK-hat / dV
                       // rows of key N - 1 here ([planes][n_blk][2][D] fp32)
  void* qhat_f;        // non-null (fp16 logits): fp16 of Q-hat * scale * log2(e),
                       // [planes][N][D], written by the dQ kernel's first pass and
                       // staged by the dK/dV (or key-tile) kernel
  float* row_stat;     // non-null: per query row {|dO|_2, max |Q-hat * scale * log2(e)|}
                       // [planes * N][2], written by the dQ kernel's first pass; the
                       // key-tile kernel (bwd_keys.hip) then replaces the dK/dV kernel
  // Stored-dS backward (bwd_ds.hip); ds_t non-null selects it in the key tiles.
  void* ds_t;          // fp16 sig * dS^T of the key tiles: [planes][n_kt * 128][nqp]
  void* khat;          // fp16 K-hat * fk of the key tiles: [planes][n_kt * 128][D]
  int* kexp;           // per key tile: log2 of 1 / (sig * fk), [planes][n_kt]
  float* dslast;       // non-null: dS of the lone key N - 1 per query row, [planes][N]
  int nqp;             // dS^T row pitch in elements (N rounded up to 64)
  int n_kt;            // key tiles per plane
};

// Launch shapes picked by the tile table (api.hip).
enum BwdVariant : int {
  BWD_FUSED = 0,    // one workgroup per plane: dK, dV and dQ in one pass (N <= 256)
  BWD_SPLIT = 1,    // dQ kernel (Q-outer, also writes delta) + dK/dV kernel (KV-outer)
  BWD_SPLIT16 = 2,  // dQ kernel + key-tile kernel, both with fp16 dS products
                    // (bwd_keys.hip; with vector access to every tensor, else BWD_SPLIT)
  BWD_DS = 3,       // row pass + key tiles that store dS + dQ as one GEMM over it
                    // (bwd_ds.hip; with vector access to every tensor, else BWD_SPLIT16)
};

// Launchers: return hipSuccess or the launch error.  io/ct are DT_* codes.
hipError_t launch_fwd(const FwdParams& p, int io, int ct, int D, hipStream_t st);
hipError_t launch_bwd_pre(const BwdParams& p, int io, int D, hipStream_t st);
hipError_t launch_bwd_dq(const BwdParams& p, int io, int ct, int D, bool write_delta,
                         hipStream_t st);
hipError_t launch_bwd_dkdv(const BwdParams& p, int io, int ct, int D, hipStream_t st);
// One-pass backward (bwd_fused.hip): D = 64, N <= bwd_fused_rows(), ct bf16 or fp16.
hipError_t launch_bwd_fused(const BwdParams& p, int io, int ct, hipStream_t st);
hipError_t launch_rope_pack(const float* cosp, int64_t cs0, int64_t cs1, const float* sinp,
                            int64_t ss0, int64_t ss1, int n_pos, int d2, float* out,
                            hipStream_t st);

// Forward for ViT-sized planes (fwd_plane.hip): one wave per (b, h) plane
// with the plane's K-hat and V^T held in registers.  fwd_plane_ok: 16-bit
// I/O with the same compute type, head_dim 64, 193 <= N <= 208 and vector
// access to every tensor.  Covers whole planes (no tail rows).
bool fwd_plane_ok(int io, int ct, int D, int N, int has_cls, bool vec);
int fwd_plane_rows();
int fwd_plane_threads();
hipError_t launch_fwd_plane(const FwdParams& p, int io, hipStream_t st);

// Tail rows (tail.hip): when 0 < N % block_rows <= kTailMaxRows and N >= block_rows,
// the block kernels cover the full blocks only and these kernels compute the
// last tail_rows(N, block_rows) rows (forward: O, LSE; rows: dQ and, with
// write_delta, delta; keys: dK, dV) -- rows [row0, N) of every plane.
constexpr int kTailMaxRows = 8;
int tail_rows(int N, int block_rows);
hipError_t launch_fwd_tail(const FwdParams& p, int io, int D, int row0, hipStream_t st);
hipError_t launch_bwd_tail_rows(const BwdParams& p, int io, int D, int row0, bool write_delta,
                                hipStream_t st);
hipError_t launch_bwd_tail_keys(const BwdParams& p, int io, int D, int key0, hipStream_t st);
// Key N - 1 from the dQ kernel's per-tile partial rows (p.xk_ws, nparts per
// plane) instead of launch_bwd_tail_keys; D = 128 or 256, 16-bit I/O.
hipError_t launch_bwd_tail_key_merge(const BwdParams& p, int io, int D, int nparts, hipStream_t st);
// Key tiles with fp16 dS products (bwd_keys.hip): dK and dV of p.n_blk
// 128-key tiles per plane, in place of launch_bwd_dkdv, for 16-bit I/O, bf16
// compute, head_dim 128 and vector access to every tensor; needs p.qhat_f and
// p.row_stat (and delta) from the dQ kernel's pass before it.
constexpr int kKeysRows = 128;
hipError_t launch_bwd_keys(const BwdParams& p, int io, hipStream_t st);
// Stored-dS backward (bwd_ds.hip), the key tiles' shapes: the row pass
// (delta, p.qhat_f, p.row_stat and, with p.dslast, the lone last key's dS and
// partial dK-hat / dV rows into p.xk_ws, one pair per row tile) before the
// key tiles, and the dQ GEMM over their stored dS after them (with p.dslast
// it also sums those partial rows into the last key's dK and dV).
constexpr int kDsPrepRows = 64;     // query rows per row-pass workgroup
constexpr int kDsQueryRows = 256;   // query rows per dQ GEMM workgroup
constexpr int kDsMaxKeyTiles = 256;  // key tiles per plane (N < 32768, from the 32-bit dS^T offsets)
hipError_t launch_bwd_ds_prep(const BwdParams& p, int io, hipStream_t st);
hipError_t launch_bwd_ds_dq(const BwdParams& p, int io, hipStream_t st);

// Whether the forward block kernel computes a single tail row itself
// (FwdParams::x_rows = 1) instead of launch_fwd_tail: fp16 logit operands with
// vector access (vec: every tensor of the call allows it).
bool fwd_folds_tail(int io, int ct, int D, bool vec);
// The same for the dQ kernel's tail row (vec: K and V allow vector access),
// instead of launch_bwd_tail_rows.  (The dK/dV kernel keeps its tail kernel:
// the tail key's VALU work lengthens every query stage of its tile by more
// than the tail kernel costs.)
bool bwd_folds_tail(int io, int ct, int D, bool vec);

// fp16 logit operands and split dS: bf16 compute at head_dim >= 128.
// Rounding the rotated Q / K rows to bf16 before the logits product is the
// dominant error of bf16 attention there (long, wide planes with large
// logits).  Those kernels round them to fp16 instead (3 more mantissa bits;
// operands beyond fp16's range are handled by a rescaled second pass, see
// f16_fit in common.h) and take the dQ / dK products from dS = hi + lo (two
// bf16 parts).  fp16 compute is fp16 throughout, and fp32 compute splits
// every operand anyway.
constexpr bool f16_logits(int ct, int D) { return ct == 2 /* DT_BF16 */ && D >= 128; }
// With those logits the next dQ / dK error term is delta = rowsum(dO * O)
// taken from the bf16-stored O.  bf16 I/O then also stores O's rounding
// residual bf16(O - bf16(O)) (when the caller provides the buffer), and the
// backward takes delta from O + residual.
constexpr bool o_residual(int io, int ct, int D) { return io == 2 && f16_logits(ct, D); }

// Workgroups for a persistent kernel: min(items, CUs x resident workgroups per
// CU), with `dyn_lds` bytes of dynamic LDS per workgroup; <= 0 on a HIP error.
int persistent_grid(const void* kernel, int block_threads, int items, size_t dyn_lds = 0);

// Rows of q (fwd, dq) or kv (dk/dv) one work item / workgroup covers.
int fwd_block_rows(int D, int io, int ct);
int fwd_threads(int D);
int bwd_dq_block_rows(int D, int ct);
int bwd_dkdv_block_rows(int D, int ct);
int bwd_dkdv_threads(int D, int ct);
int bwd_fused_rows();

}  // namespace farope
