// C-ABI layer: argument validation, the tile table, and kernel dispatch.
// Declarations and per-function reference citations: include/farope.h.
#include "farope.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <unordered_map>

#include "params.h"

using namespace farope;

// Workspace of farope_attn_bwd_noalloc: the split backward's delta rows (fp32,
// one per query row of the call) and, for a lone last key, the dQ tiles'
// partial dK / dV rows after them (bwd_ws_elems <= FAROPE_NOALLOC_MAX_ROWS,
// 16 MiB).
// The runtime gives every device its own copy when it loads the code object,
// held until the process ends.  In host code this name is only a handle for
// hipGetSymbolAddress: kernels receive the device address it returns.
static __device__ __align__(256) float scratch[FAROPE_NOALLOC_MAX_ROWS];

namespace farope {

// Resident-capacity query for persistent kernels, cached per (device, kernel).
int persistent_grid(const void* kernel, int block_threads, int items, size_t dyn_lds) {
  static std::mutex mu;
  static std::unordered_map<uint64_t, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  const uint64_t key = ((reinterpret_cast<uint64_t>(kernel) << 8) ^ (uint64_t)(dev & 0xff)) +
                       ((uint64_t)dyn_lds << 48);
  int cap = 0;
  {
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) cap = it->second;
  }
  if (cap == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block_threads, dyn_lds) !=
        hipSuccess)
      return -1;
    cap = cus * (per_cu > 0 ? per_cu : 1);
    std::lock_guard<std::mutex> lock(mu);
    cache[key] = cap;
  }
  return items < cap ? items : cap;
}

}  // namespace farope

namespace {

constexpr int kPlaneMaxN = 256;   // fused / plane-resident kernels hold <= 256 rows of a plane

int elem_size(int dt) { return dt == FAROPE_F32 ? 4 : 2; }

bool dtype_ok(int dt) { return dt == FAROPE_F32 || dt == FAROPE_F16 || dt == FAROPE_BF16; }

int check_desc(const farope_attn_desc* d) {
  if (!d) return FAROPE_ERR_NULL;
  if (d->batch <= 0 || d->heads <= 0) return FAROPE_ERR_SHAPE;
  if ((int64_t)d->batch * d->heads > (int64_t)(1 << 30)) return FAROPE_ERR_SHAPE;
  if (d->head_dim <= 0 || d->head_dim % 4 != 0) return FAROPE_ERR_HEAD_DIM;
  if (d->head_dim != 32 && d->head_dim != 64 && d->head_dim != 128 && d->head_dim != 256)
    return FAROPE_ERR_HEAD_DIM;
  if (d->has_cls != 0 && d->has_cls != 1) return FAROPE_ERR_SEQ_LEN;
  if (d->n_pos < 1 || d->seq_len != d->n_pos + d->has_cls) return FAROPE_ERR_SEQ_LEN;
  if (!dtype_ok(d->io_dtype) || !dtype_ok(d->compute_dtype)) return FAROPE_ERR_DTYPE;
  return FAROPE_OK;
}

// The packed table a call passes must be the one of its geometry:
// farope_rope_packed_elems(n_pos, head_dim / 2) fp32 values.
int check_table(const farope_attn_desc* d, const float* rope, size_t elems) {
  if (!rope) return FAROPE_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(rope) % 16) return FAROPE_ERR_ALIGN;
  if (elems != (size_t)(d->n_pos + 1) * (size_t)d->head_dim) return FAROPE_ERR_TABLE;
  return FAROPE_OK;
}

int check_ptr(const void* p, int es) {
  if (!p) return FAROPE_ERR_NULL;
  if (reinterpret_cast<uintptr_t>(p) % es) return FAROPE_ERR_ALIGN;
  return FAROPE_OK;
}

// 16-byte vector path allowed: unit channel stride and 16-byte aligned rows.
// 16-byte vector access: unit d-stride, 16-byte aligned base and strides, a
// non-negative row stride, and every byte offset inside one (b, h) plane
// (row n, channel d) below 2^31, so kernels can address a plane as 64-bit
// base + 32-bit lane offset.  The bound also covers the kRowPad rows past
// the plane that the kernels address unconditionally (their blocks of up to
// 256 rows end past N): those offsets must stay below 2^31 too, so that they
// fall outside the descriptor range (loads read 0, stores are dropped)
// instead of wrapping around to a row of the plane.
constexpr int kRowPad = 256;
int vec_ok(const void* p, const int64_t s[4], int es, int n_rows, int head_dim) {
  if (s[3] != 1) return 0;
  if (reinterpret_cast<uintptr_t>(p) % 16) return 0;
  for (int i = 0; i < 3; ++i)
    if ((s[i] * es) % 16 != 0) return 0;
  if (s[2] < 0) return 0;   // lane offsets are unsigned
  if ((int64_t)(n_rows - 1 + kRowPad) * s[2] + head_dim >= ((int64_t)1 << 31) / es) return 0;
  return 1;
}

// Written tensors additionally need rows that do not overlap (row stride >=
// head_dim): the kernels then store rows >= N unconditionally and rely on
// the descriptor range to drop them.
int vec_out_ok(const void* p, const int64_t s[4], int es, int n_rows, int head_dim) {
  return vec_ok(p, s, es, n_rows, head_dim) && s[2] >= head_dim;
}

void copy4(int64_t dst[4], const int64_t src[4]) {
  for (int i = 0; i < 4; ++i) dst[i] = src[i];
}

// The one-pass backward keeps bf16/fp16 tiles of the plane in LDS; fp32
// compute (twice the bytes) takes the split path.
bool bwd_fused(const farope_attn_desc* d) {
  return d->head_dim == 64 && d->seq_len <= bwd_fused_rows() && d->compute_dtype != FAROPE_F32;
}

// The plane forward (fwd_plane.hip): one wave per ViT-sized plane, when every
// tensor allows vector access (tile_config, which sees no tensors, assumes it).
bool fwd_plane(const farope_attn_desc* d, bool vec) {
  return fwd_plane_ok(d->io_dtype, d->compute_dtype, d->head_dim, d->seq_len, d->has_cls, vec);
}

int cdiv(int a, int b) { return (a + b - 1) / b; }

int fill_common(BwdParams& p, const farope_attn_desc* d, const float* rope) {
  p.rope = rope;
  p.B = d->batch;
  p.H = d->heads;
  p.N = d->seq_len;
  p.has_cls = d->has_cls;
  p.scale = d->softmax_scale;
  p.scale_log2 = d->softmax_scale * 1.4426950408889634f;
  return FAROPE_OK;
}

#define FAROPE_TRY(expr)            \
  do {                              \
    const int rc__ = (expr);        \
    if (rc__ != FAROPE_OK) return rc__; \
  } while (0)

int launch_rc(hipError_t e) { return e == hipSuccess ? FAROPE_OK : FAROPE_ERR_LAUNCH; }

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
constexpr int kMaxDevices = 64;
constexpr int64_t kScratchFloats = FAROPE_NOALLOC_MAX_ROWS;

int scratch_ptr(float** out) {
  static std::mutex mu;
  static float* ptrs[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return FAROPE_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return FAROPE_ERR_LAUNCH;
    ptrs[dev] = static_cast<float*>(ptr);
  }
  *out = ptrs[dev];
  return FAROPE_OK;
}

// Rows left to the tail kernels (0: none).  Their grid holds one workgroup
// per (plane, row), so it must stay within the 2^31 - 1 grid limit.
int tail_of(int planes, int N, int rows) {
  const int t = tail_rows(N, rows);
  return (int64_t)planes * t <= INT32_MAX ? t : 0;
}

// Block count for N rows in blocks of `rows`; with a tail, full blocks only.
int main_blocks(int planes, int N, int rows) {
  return tail_of(planes, N, rows) ? N / rows : cdiv(N, rows);
}

// dQ block kernel (+ the tail rows kernel); with write_delta both write delta
int dq_pass(BwdParams p, const farope_attn_desc* d, bool write_delta, hipStream_t st) {
  const int D = d->head_dim, rows = bwd_dq_block_rows(D, d->compute_dtype);
  const int tail = tail_of(p.B * p.H, p.N, rows);
  p.n_blk = main_blocks(p.B * p.H, p.N, rows);
  p.x_rows = tail == 1 && bwd_folds_tail(d->io_dtype, d->compute_dtype, D, p.vec_k && p.vec_v);
  FAROPE_TRY(launch_rc(launch_bwd_dq(p, d->io_dtype, d->compute_dtype, D, write_delta, st)));
  if (tail && !p.x_rows)
    FAROPE_TRY(launch_rc(launch_bwd_tail_rows(p, d->io_dtype, D, p.N - tail, write_delta, st)));
  return FAROPE_OK;
}

// dK/dV block kernel (+ the tail keys kernel, or the merge of the dQ tiles'
// partial rows of the last key when dq_pass wrote them to p.xk_ws)
int dkdv_pass(BwdParams p, const farope_attn_desc* d, hipStream_t st) {
  const int D = d->head_dim, rows = bwd_dkdv_block_rows(D, d->compute_dtype);
  const int tail = tail_of(p.B * p.H, p.N, rows);
  p.n_blk = main_blocks(p.B * p.H, p.N, rows);
  if (p.row_stat)   // the dQ pass wrote the statistics the key tiles need
    FAROPE_TRY(launch_rc(launch_bwd_keys(p, d->io_dtype, st)));
  else
    FAROPE_TRY(launch_rc(launch_bwd_dkdv(p, d->io_dtype, d->compute_dtype, D, st)));
  if (tail && p.xk_ws) {
    const int nparts = main_blocks(p.B * p.H, p.N, bwd_dq_block_rows(D, d->compute_dtype));
    FAROPE_TRY(launch_rc(launch_bwd_tail_key_merge(p, d->io_dtype, D, nparts, st)));
  } else if (tail) {
    FAROPE_TRY(launch_rc(launch_bwd_tail_keys(p, d->io_dtype, D, p.N - tail, st)));
  }
  return FAROPE_OK;
}

// Whether the one-call backward takes the last key's dK / dV from the dQ
// tiles' partial rows: one row left past both kernels' full blocks, fp16
// logit operands (vec: K and V allow vector access, as the dQ kernel's
// folded-row instantiation needs).  The workspace size below assumes vec.
bool key_from_dq(const farope_attn_desc* d, bool vec) {
  const int D = d->head_dim, planes = d->batch * d->heads, N = d->seq_len;
  return tail_of(planes, N, bwd_dq_block_rows(D, d->compute_dtype)) == 1 &&
         tail_of(planes, N, bwd_dkdv_block_rows(D, d->compute_dtype)) == 1 &&
         bwd_folds_tail(d->io_dtype, d->compute_dtype, D, vec);
}

// Whether the dQ kernel can hand its rotated Q rows to the dK/dV kernel
// (fp16 logit operands; every row is a dQ-tile row: no tail, or the folded
// one).  The dK/dV kernel then also needs vector access to dO (checked at
// the call).
bool qhat_possible(const farope_attn_desc* d) {
  const int D = d->head_dim, planes = d->batch * d->heads, N = d->seq_len;
  if (bwd_fused(d) || d->io_dtype == FAROPE_F32 || !f16_logits(d->compute_dtype, D)) return false;
  const int t = tail_of(planes, N, bwd_dq_block_rows(D, d->compute_dtype));
  return t == 0 || (t == 1 && bwd_folds_tail(d->io_dtype, d->compute_dtype, D, true));
}

// Workspace of the split backward, in fp32 elements: the delta rows, then
// (key_from_dq) one dK-hat / dV row pair per dQ tile, then (with_hat and
// qhat_possible, from a 256-byte boundary) the rotated Q rows in fp16.
struct BwdWs {
  int64_t keys, hat, total;   // offsets of the key rows and of the rotated rows; size
};
BwdWs bwd_ws(const farope_attn_desc* d, bool with_hat) {
  const int64_t planes = (int64_t)d->batch * d->heads, rows = planes * d->seq_len;
  if (bwd_fused(d)) return BwdWs{0, 0, 0};   // the one-pass kernel keeps delta on chip
  BwdWs w{rows, 0, rows};
  if (key_from_dq(d, true)) {
    const int nb = main_blocks((int)planes, d->seq_len, bwd_dq_block_rows(d->head_dim, d->compute_dtype));
    w.total += planes * nb * 2 * d->head_dim;
  }
  if (with_hat && qhat_possible(d)) {
    w.hat = (w.total + 63) & ~int64_t(63);
    w.total = w.hat + rows * d->head_dim / 2;   // [planes][N][D] fp16
  }
  return w;
}
int64_t bwd_ws_elems(const farope_attn_desc* d) { return bwd_ws(d, false).total; }

// Key tiles with fp16 dS products (bwd_keys.hip) in place of the dK/dV
// kernel: 16-bit I/O, bf16 compute, head_dim 128, with the dQ pass's rotated
// Q rows (the call also needs vector access to every tensor, checked there).
bool keys_possible(const farope_attn_desc* d) {
  return qhat_possible(d) && d->head_dim == kKeysRows && d->compute_dtype == FAROPE_BF16;
}
// Caller workspace of the split path with key tiles: bwd_ws, then (from a
// 256-byte boundary) one {|dO|_2, max |Q-hat c2|} pair per query row.
int64_t stat_offset(const farope_attn_desc* d) { return (bwd_ws(d, true).total + 63) & ~int64_t(63); }
int64_t split_caller_ws(const farope_attn_desc* d) {
  if (!keys_possible(d)) return bwd_ws(d, true).total;
  return stat_offset(d) + 2 * (int64_t)d->batch * d->heads * d->seq_len;
}

// The stored-dS backward (bwd_ds.hip): the key tiles' shapes (16-bit I/O, bf16
// compute, head_dim 128) with at most one key past the full key tiles, and a
// dS^T plane of at most 16 Q planes (N up to about 2k; its workspace grows
// with N^2, the split path's with N).  (Vector access to every tensor is
// checked at the call.)
constexpr int kDsD = 128;
int ds_pitch(int N) { return (N + 63) & ~63; }   // 128-byte rows
bool ds_possible(const farope_attn_desc* d) {
  if (bwd_fused(d) || d->io_dtype == FAROPE_F32 || d->compute_dtype != FAROPE_BF16 || d->head_dim != kDsD)
    return false;
  const int planes = d->batch * d->heads, N = d->seq_len;
  if (tail_of(planes, N, kKeysRows) > 1) return false;
  const int64_t n_kt = main_blocks(planes, N, kKeysRows), kp = n_kt * kKeysRows;
  return n_kt <= kDsMaxKeyTiles && kp * ds_pitch(N) <= 16 * (int64_t)N * kDsD;
}
// Its workspace, in fp32 elements, each part from a 256-byte boundary: delta
// rows; (lone last key) one partial dK-hat / dV row pair per row-pass tile;
// fp16 Q-hat * c2 rows; row statistics; (lone last key) its dS per row; the
// key tiles' exponents (int32); their fp16 K-hat * fk rows; their fp16
// sig dS^T rows.
struct DsWs {
  int64_t xk, hat, stat, dsl, kexp, khat, dst, total;
};
DsWs ds_ws(const farope_attn_desc* d) {
  const int planes = d->batch * d->heads, N = d->seq_len;
  const int64_t rows = (int64_t)planes * N;
  const bool last = tail_of(planes, N, kKeysRows) == 1;
  const int64_t n_kt = main_blocks(planes, N, kKeysRows), kp = n_kt * kKeysRows;
  const int64_t n_pt = cdiv(N, kDsPrepRows);
  auto al = [](int64_t x) { return (x + 63) & ~int64_t(63); };
  DsWs w{};
  w.xk = al(rows);
  w.hat = al(w.xk + (last ? planes * n_pt * 2 * kDsD : 0));
  w.stat = al(w.hat + rows * kDsD / 2);
  w.dsl = al(w.stat + 2 * rows);
  w.kexp = al(w.dsl + (last ? rows : 0));
  w.khat = al(w.kexp + planes * n_kt);
  w.dst = al(w.khat + planes * kp * kDsD / 2);
  w.total = w.dst + planes * kp * ds_pitch(N) / 2;
  return w;
}

// Caller workspace of farope_attn_bwd: enough for whichever path the call
// takes.
int64_t bwd_caller_ws(const farope_attn_desc* d) {
  const int64_t s = split_caller_ws(d);
  if (!ds_possible(d)) return s;
  const int64_t t = ds_ws(d).total;
  return t > s ? t : s;
}

// Stored-dS backward: row pass, key tiles (storing dS), dQ GEMM (which also
// merges the lone last key's partial dK / dV rows).
int ds_pass(BwdParams p, const farope_attn_desc* d, float* ws, hipStream_t st) {
  const DsWs w = ds_ws(d);
  const int planes = p.B * p.H, N = p.N;
  const bool last = tail_of(planes, N, kKeysRows) == 1;
  p.qhat_f = ws + w.hat;
  p.row_stat = ws + w.stat;
  p.xk_ws = last ? ws + w.xk : nullptr;
  p.dslast = last ? ws + w.dsl : nullptr;
  p.kexp = reinterpret_cast<int*>(ws + w.kexp);
  p.khat = ws + w.khat;
  p.ds_t = ws + w.dst;
  p.nqp = ds_pitch(N);
  p.n_kt = main_blocks(planes, N, kKeysRows);
  FAROPE_TRY(launch_rc(launch_bwd_ds_prep(p, d->io_dtype, st)));
  p.n_blk = p.n_kt;
  FAROPE_TRY(launch_rc(launch_bwd_keys(p, d->io_dtype, st)));
  return launch_rc(launch_bwd_ds_dq(p, d->io_dtype, st));
}

int bwd_impl(const farope_attn_desc* desc, const void* q, const int64_t q_stride[4],
             const void* k, const int64_t k_stride[4], const void* v, const int64_t v_stride[4],
             const void* o, const int64_t o_stride[4], const void* o_res, const void* dout,
             const int64_t dout_stride[4], const float* lse, const float* rope_packed, size_t rope_elems, void* dq,
             const int64_t dq_stride[4], void* dk, const int64_t dk_stride[4], void* dv,
             const int64_t dv_stride[4], float* delta_ws, bool static_ws, void* stream) {
  FAROPE_TRY(check_desc(desc));
  if (!q_stride || !k_stride || !v_stride || !o_stride || !dout_stride || !dq_stride ||
      !dk_stride || !dv_stride)
    return FAROPE_ERR_NULL;
  const int es = elem_size(desc->io_dtype);
  FAROPE_TRY(check_ptr(q, es));
  FAROPE_TRY(check_ptr(k, es));
  FAROPE_TRY(check_ptr(v, es));
  FAROPE_TRY(check_ptr(o, es));
  FAROPE_TRY(check_ptr(dout, es));
  FAROPE_TRY(check_ptr(dq, es));
  FAROPE_TRY(check_ptr(dk, es));
  FAROPE_TRY(check_ptr(dv, es));
  FAROPE_TRY(check_ptr(lse, 4));
  FAROPE_TRY(check_table(desc, rope_packed, rope_elems));
  const bool fused = bwd_fused(desc);
  if (!fused) {
    if (static_ws) {
      // the split path's delta rows go to this device's static scratch array
      if (bwd_ws_elems(desc) > kScratchFloats) return FAROPE_ERR_SCRATCH;
      FAROPE_TRY(scratch_ptr(&delta_ws));
    } else {
      FAROPE_TRY(check_ptr(delta_ws, 4));
    }
  }
  if (o_res) FAROPE_TRY(check_ptr(o_res, 16));
  BwdParams p = {};
  fill_common(p, desc, rope_packed);
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout;
  p.o_res = o_residual(desc->io_dtype, desc->compute_dtype, desc->head_dim) ? o_res : nullptr;
  p.dq = dq; p.dk = dk; p.dv = dv;
  p.lse = lse; p.delta = delta_ws;
  copy4(p.sq, q_stride); copy4(p.sk, k_stride); copy4(p.sv, v_stride); copy4(p.so, o_stride);
  copy4(p.sdo, dout_stride); copy4(p.sdq, dq_stride); copy4(p.sdk, dk_stride);
  copy4(p.sdv, dv_stride);
  p.vec_q = vec_ok(q, q_stride, es, desc->seq_len, desc->head_dim);
  p.vec_k = vec_ok(k, k_stride, es, desc->seq_len, desc->head_dim);
  p.vec_v = vec_ok(v, v_stride, es, desc->seq_len, desc->head_dim);
  p.vec_o = vec_ok(o, o_stride, es, desc->seq_len, desc->head_dim);
  p.vec_do = vec_ok(dout, dout_stride, es, desc->seq_len, desc->head_dim);
  p.vec_dq = vec_out_ok(dq, dq_stride, es, desc->seq_len, desc->head_dim);
  p.vec_dk = vec_out_ok(dk, dk_stride, es, desc->seq_len, desc->head_dim);
  p.vec_dv = vec_out_ok(dv, dv_stride, es, desc->seq_len, desc->head_dim);
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const int D = desc->head_dim;
  if (fused) {
    p.n_blk = 1;
    return launch_rc(launch_bwd_fused(p, desc->io_dtype, desc->compute_dtype, st));
  }
  // the stored-dS backward (the static workspace only when all of it fits)
  if (ds_possible(desc) && p.vec_q && p.vec_k && p.vec_v && p.vec_o && p.vec_do && p.vec_dq &&
      p.vec_dk && p.vec_dv && reinterpret_cast<uintptr_t>(delta_ws) % 16 == 0 &&
      (!static_ws || ds_ws(desc).total <= kScratchFloats))
    return ds_pass(p, desc, delta_ws, st);
  // dQ (and delta, which the dK/dV pass reads for every row) before dK / dV
  if (key_from_dq(desc, p.vec_k && p.vec_v))
    p.xk_ws = delta_ws + (int64_t)desc->batch * desc->heads * desc->seq_len;
  // the rotated Q rows go to the workspace too: always for a caller
  // workspace (sized by farope_attn_bwd_workspace_elems), for the static one
  // when they fit
  if (qhat_possible(desc) && p.vec_q && p.vec_do &&
      (!static_ws || bwd_ws(desc, true).total <= kScratchFloats)) {
    const BwdWs w = bwd_ws(desc, true);
    const int tq = tail_of(p.B * p.H, p.N, bwd_dq_block_rows(D, desc->compute_dtype));
    float* hat = delta_ws + w.hat;
    if ((tq == 0 || bwd_folds_tail(desc->io_dtype, desc->compute_dtype, D, p.vec_k && p.vec_v)) &&
        reinterpret_cast<uintptr_t>(hat) % 16 == 0)
      p.qhat_f = hat;
  }
  // the key tiles with fp16 dS products take the dK/dV pass (the static
  // workspace only when all of it fits)
  if (p.qhat_f && keys_possible(desc) && p.vec_k && p.vec_v && p.vec_o && p.vec_dq && p.vec_dk &&
      p.vec_dv && (!static_ws || split_caller_ws(desc) <= kScratchFloats))
    p.row_stat = delta_ws + stat_offset(desc);
  FAROPE_TRY(dq_pass(p, desc, true, st));
  return dkdv_pass(p, desc, st);
}

}  // namespace

extern "C" {

int farope_abi_version(void) { return FAROPE_ABI_VERSION; }

const char* farope_strerror(int status) {
  switch (status) {
    case FAROPE_OK: return "success";
    case FAROPE_ERR_NULL: return "farope: a required pointer is NULL";
    case FAROPE_ERR_HEAD_DIM:
      return "farope: unsupported head_dim (must be divisible by 4; kernels exist for 32, 64, 128 and 256)";
    case FAROPE_ERR_SEQ_LEN: return "farope: seq_len must equal n_pos + has_cls";
    case FAROPE_ERR_DTYPE: return "farope: unsupported dtype (float32, float16, bfloat16)";
    case FAROPE_ERR_TABLE:
      return "farope: RoPE table geometry does not match the call (rope_elems must be farope_rope_packed_elems(n_pos, head_dim / 2))";
    case FAROPE_ERR_SHAPE: return "farope: batch/heads must be positive and B*H <= 2^30";
    case FAROPE_ERR_LAUNCH: return "farope: HIP kernel launch failed";
    case FAROPE_ERR_ALIGN: return "farope: pointer not aligned to its element size";
    case FAROPE_ERR_SCRATCH:
      return "farope: the backward workspace (farope_attn_bwd_workspace_elems) exceeds the static workspace of farope_attn_bwd_noalloc "
             "(FAROPE_NOALLOC_MAX_ROWS = 4194304); use farope_attn_bwd with a caller workspace";
    default: return "farope: unknown status";
  }
}

size_t farope_rope_packed_elems(int32_t n_pos, int32_t d2) {
  if (n_pos < 0 || d2 < 0) return 0;
  return (size_t)(n_pos + 1) * (size_t)d2 * 2;
}

int farope_rope_pack(const float* cosp, int64_t cos_stride0, int64_t cos_stride1,
                     const float* sinp, int64_t sin_stride0, int64_t sin_stride1,
                     int32_t n_pos, int32_t d2, float* packed, void* stream) {
  if (!cosp || !sinp || !packed) return FAROPE_ERR_NULL;
  if (n_pos < 1 || d2 < 1 || d2 % 2 != 0) return FAROPE_ERR_TABLE;
  if (reinterpret_cast<uintptr_t>(packed) % 16) return FAROPE_ERR_ALIGN;
  return launch_rc(launch_rope_pack(cosp, cos_stride0, cos_stride1, sinp, sin_stride0,
                                    sin_stride1, n_pos, d2, packed,
                                    static_cast<hipStream_t>(stream)));
}

int farope_tile_config(const farope_attn_desc* desc, int32_t which, int32_t out[4]) {
  FAROPE_TRY(check_desc(desc));
  if (!out) return FAROPE_ERR_NULL;
  const int D = desc->head_dim, N = desc->seq_len;
  if (which == 0) {
    if (fwd_plane(desc, true)) {
      out[0] = 1;
      out[1] = fwd_plane_rows();
      out[2] = 1;
      out[3] = fwd_plane_threads();
      return FAROPE_OK;
    }
    const int rows = fwd_block_rows(D, desc->io_dtype, desc->compute_dtype);
    out[0] = 0;
    out[1] = rows;
    out[2] = main_blocks(desc->batch * desc->heads, N, rows);
    out[3] = fwd_threads(D);
  } else {
    const bool fu = bwd_fused(desc);
    out[0] = fu ? BWD_FUSED : ds_possible(desc) ? BWD_DS : keys_possible(desc) ? BWD_SPLIT16 : BWD_SPLIT;
    out[1] = fu ? bwd_fused_rows() : bwd_dkdv_block_rows(D, desc->compute_dtype);
    out[2] = fu ? cdiv(N, out[1]) : main_blocks(desc->batch * desc->heads, N, out[1]);
    out[3] = fu ? 512 : bwd_dkdv_threads(D, desc->compute_dtype);
  }
  return FAROPE_OK;
}

size_t farope_attn_bwd_workspace_elems(const farope_attn_desc* desc) {
  if (check_desc(desc) != FAROPE_OK) return 0;
  return (size_t)bwd_caller_ws(desc);
}

size_t farope_attn_residual_elems(const farope_attn_desc* desc) {
  if (check_desc(desc) != FAROPE_OK) return 0;
  if (!o_residual(desc->io_dtype, desc->compute_dtype, desc->head_dim)) return 0;
  return (size_t)desc->batch * desc->heads * desc->seq_len * desc->head_dim;
}

int farope_attn_fwd(const farope_attn_desc* desc, const void* q, const int64_t q_stride[4],
                    const void* k, const int64_t k_stride[4], const void* v,
                    const int64_t v_stride[4], const float* rope_packed, size_t rope_elems, void* o,
                    const int64_t o_stride[4], void* o_res, float* lse, void* stream) {
  FAROPE_TRY(check_desc(desc));
  if (!q_stride || !k_stride || !v_stride || !o_stride) return FAROPE_ERR_NULL;
  const int es = elem_size(desc->io_dtype);
  FAROPE_TRY(check_ptr(q, es));
  FAROPE_TRY(check_ptr(k, es));
  FAROPE_TRY(check_ptr(v, es));
  FAROPE_TRY(check_ptr(o, es));
  FAROPE_TRY(check_ptr(lse, 4));
  FAROPE_TRY(check_table(desc, rope_packed, rope_elems));
  if (o_res) FAROPE_TRY(check_ptr(o_res, 16));

  FwdParams p;
  p.q = q; p.k = k; p.v = v; p.o = o; p.lse = lse;
  p.o_res = o_residual(desc->io_dtype, desc->compute_dtype, desc->head_dim) ? o_res : nullptr;
  copy4(p.sq, q_stride); copy4(p.sk, k_stride); copy4(p.sv, v_stride); copy4(p.so, o_stride);
  p.rope = rope_packed;
  p.B = desc->batch; p.H = desc->heads; p.N = desc->seq_len; p.has_cls = desc->has_cls;
  p.scale_log2 = desc->softmax_scale * 1.4426950408889634f;
  p.vec_q = vec_ok(q, q_stride, es, desc->seq_len, desc->head_dim);
  p.vec_k = vec_ok(k, k_stride, es, desc->seq_len, desc->head_dim);
  p.vec_v = vec_ok(v, v_stride, es, desc->seq_len, desc->head_dim);
  p.vec_o = vec_out_ok(o, o_stride, es, desc->seq_len, desc->head_dim);
  const bool vec = p.vec_q && p.vec_k && p.vec_v && p.vec_o;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  if (fwd_plane(desc, vec)) {
    p.n_blk = 1;
    p.n_items = p.B * p.H;
    p.x_rows = 0;
    return launch_rc(launch_fwd_plane(p, desc->io_dtype, st));
  }
  const int rows = fwd_block_rows(desc->head_dim, desc->io_dtype, desc->compute_dtype);
  const int tail = tail_of(p.B * p.H, p.N, rows);
  p.n_blk = main_blocks(p.B * p.H, p.N, rows);
  p.n_items = p.B * p.H * p.n_blk;
  p.x_rows = tail == 1 && fwd_folds_tail(desc->io_dtype, desc->compute_dtype, desc->head_dim, vec);
  FAROPE_TRY(launch_rc(launch_fwd(p, desc->io_dtype, desc->compute_dtype, desc->head_dim, st)));
  if (tail && !p.x_rows)
    FAROPE_TRY(launch_rc(launch_fwd_tail(p, desc->io_dtype, desc->head_dim, p.N - tail, st)));
  return FAROPE_OK;
}

int farope_attn_bwd_preprocess(const farope_attn_desc* desc, const void* o,
                               const int64_t o_stride[4], const void* o_res, const void* dout,
                               const int64_t dout_stride[4], float* delta, void* stream) {
  FAROPE_TRY(check_desc(desc));
  if (!o_stride || !dout_stride) return FAROPE_ERR_NULL;
  const int es = elem_size(desc->io_dtype);
  FAROPE_TRY(check_ptr(o, es));
  FAROPE_TRY(check_ptr(dout, es));
  FAROPE_TRY(check_ptr(delta, 4));
  BwdParams p = {};
  fill_common(p, desc, nullptr);
  p.o = o; p.dout = dout; p.delta = delta;
  if (o_res) FAROPE_TRY(check_ptr(o_res, 16));
  p.o_res = o_residual(desc->io_dtype, desc->compute_dtype, desc->head_dim) ? o_res : nullptr;
  copy4(p.so, o_stride); copy4(p.sdo, dout_stride);
  p.vec_o = vec_ok(o, o_stride, es, desc->seq_len, desc->head_dim);
  p.vec_do = vec_ok(dout, dout_stride, es, desc->seq_len, desc->head_dim);
  return launch_rc(launch_bwd_pre(p, desc->io_dtype, desc->head_dim,
                                  static_cast<hipStream_t>(stream)));
}

int farope_attn_bwd_dk_dv(const farope_attn_desc* desc, const void* q, const int64_t q_stride[4],
                          const void* k, const int64_t k_stride[4], const void* v,
                          const int64_t v_stride[4], const void* dout,
                          const int64_t dout_stride[4], const float* lse, const float* delta,
                          const float* rope_packed, size_t rope_elems, void* dk, const int64_t dk_stride[4],
                          void* dv, const int64_t dv_stride[4], void* stream) {
  FAROPE_TRY(check_desc(desc));
  if (!q_stride || !k_stride || !v_stride || !dout_stride || !dk_stride || !dv_stride)
    return FAROPE_ERR_NULL;
  const int es = elem_size(desc->io_dtype);
  FAROPE_TRY(check_ptr(q, es));
  FAROPE_TRY(check_ptr(k, es));
  FAROPE_TRY(check_ptr(v, es));
  FAROPE_TRY(check_ptr(dout, es));
  FAROPE_TRY(check_ptr(dk, es));
  FAROPE_TRY(check_ptr(dv, es));
  FAROPE_TRY(check_ptr(lse, 4));
  FAROPE_TRY(check_ptr(delta, 4));
  FAROPE_TRY(check_table(desc, rope_packed, rope_elems));
  BwdParams p = {};
  fill_common(p, desc, rope_packed);
  p.q = q; p.k = k; p.v = v; p.dout = dout; p.dk = dk; p.dv = dv;
  p.lse = lse; p.delta = const_cast<float*>(delta);
  copy4(p.sq, q_stride); copy4(p.sk, k_stride); copy4(p.sv, v_stride);
  copy4(p.sdo, dout_stride); copy4(p.sdk, dk_stride); copy4(p.sdv, dv_stride);
  p.vec_q = vec_ok(q, q_stride, es, desc->seq_len, desc->head_dim);
  p.vec_k = vec_ok(k, k_stride, es, desc->seq_len, desc->head_dim);
  p.vec_v = vec_ok(v, v_stride, es, desc->seq_len, desc->head_dim);
  p.vec_do = vec_ok(dout, dout_stride, es, desc->seq_len, desc->head_dim);
  p.vec_dk = vec_out_ok(dk, dk_stride, es, desc->seq_len, desc->head_dim);
  p.vec_dv = vec_out_ok(dv, dv_stride, es, desc->seq_len, desc->head_dim);
  return dkdv_pass(p, desc, static_cast<hipStream_t>(stream));
}

int farope_attn_bwd_dq(const farope_attn_desc* desc, const void* q, const int64_t q_stride[4],
                       const void* k, const int64_t k_stride[4], const void* v,
                       const int64_t v_stride[4], const void* dout, const int64_t dout_stride[4],
                       const float* lse, const float* delta, const float* rope_packed, size_t rope_elems, void* dq,
                       const int64_t dq_stride[4], void* stream) {
  FAROPE_TRY(check_desc(desc));
  if (!q_stride || !k_stride || !v_stride || !dout_stride || !dq_stride) return FAROPE_ERR_NULL;
  const int es = elem_size(desc->io_dtype);
  FAROPE_TRY(check_ptr(q, es));
  FAROPE_TRY(check_ptr(k, es));
  FAROPE_TRY(check_ptr(v, es));
  FAROPE_TRY(check_ptr(dout, es));
  FAROPE_TRY(check_ptr(dq, es));
  FAROPE_TRY(check_ptr(lse, 4));
  FAROPE_TRY(check_ptr(delta, 4));
  FAROPE_TRY(check_table(desc, rope_packed, rope_elems));
  BwdParams p = {};
  fill_common(p, desc, rope_packed);
  p.q = q; p.k = k; p.v = v; p.dout = dout; p.dq = dq;
  p.lse = lse; p.delta = const_cast<float*>(delta);
  copy4(p.sq, q_stride); copy4(p.sk, k_stride); copy4(p.sv, v_stride);
  copy4(p.sdo, dout_stride); copy4(p.sdq, dq_stride);
  p.vec_q = vec_ok(q, q_stride, es, desc->seq_len, desc->head_dim);
  p.vec_k = vec_ok(k, k_stride, es, desc->seq_len, desc->head_dim);
  p.vec_v = vec_ok(v, v_stride, es, desc->seq_len, desc->head_dim);
  p.vec_do = vec_ok(dout, dout_stride, es, desc->seq_len, desc->head_dim);
  p.vec_dq = vec_out_ok(dq, dq_stride, es, desc->seq_len, desc->head_dim);
  return dq_pass(p, desc, false, static_cast<hipStream_t>(stream));
}

int farope_attn_bwd(const farope_attn_desc* desc, const void* q, const int64_t q_stride[4],
                    const void* k, const int64_t k_stride[4], const void* v,
                    const int64_t v_stride[4], const void* o, const int64_t o_stride[4],
                    const void* o_res, const void* dout, const int64_t dout_stride[4], const float* lse,
                    const float* rope_packed, size_t rope_elems, void* dq, const int64_t dq_stride[4], void* dk,
                    const int64_t dk_stride[4], void* dv, const int64_t dv_stride[4],
                    float* delta_ws, void* stream) {
  return bwd_impl(desc, q, q_stride, k, k_stride, v, v_stride, o, o_stride, o_res, dout, dout_stride,
                  lse, rope_packed, rope_elems, dq, dq_stride, dk, dk_stride, dv, dv_stride, delta_ws, false, stream);
}

int farope_attn_bwd_noalloc(const farope_attn_desc* desc, const void* q,
                            const int64_t q_stride[4], const void* k, const int64_t k_stride[4],
                            const void* v, const int64_t v_stride[4], const void* o,
                            const int64_t o_stride[4], const void* o_res, const void* dout,
                            const int64_t dout_stride[4], const float* lse,
                            const float* rope_packed, size_t rope_elems, void* dq, const int64_t dq_stride[4],
                            void* dk, const int64_t dk_stride[4], void* dv,
                            const int64_t dv_stride[4], void* stream) {
  return bwd_impl(desc, q, q_stride, k, k_stride, v, v_stride, o, o_stride, o_res, dout, dout_stride,
                  lse, rope_packed, rope_elems, dq, dq_stride, dk, dk_stride, dv, dv_stride, nullptr, true, stream);
}

}  // extern "C"
