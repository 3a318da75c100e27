/*
 * farope: fused 2D axial RoPE + scaled-dot-product attention (forward and
 * backward) for AMD MI355X (gfx950).  Plain C ABI: device pointers, element
 * strides and sizes only.  Every entry point enqueues work on `stream` (a
 * hipStream_t, may be NULL for the default stream), allocates nothing and
 * returns FAROPE_OK or a farope_status code; argument errors are detected
 * on the host before anything is launched.
 *
 * Reference interface replaced: the Triton launches of
 * "fa_rope_full .py" (v1kstrand/triton_fused_rope_flash_attn), cited per
 * function as FA:<line>.
 *
 * Tensor conventions: q, k, v, o, dout, dq, dk, dv are [B, H, N, D] with
 * arbitrary element strides (stride[0..3] = b, h, n, d; stride 0 allowed for
 * inputs); lse and delta are contiguous fp32 [B*H, N].
 *
 * RoPE table: every entry point that reads the packed table takes its
 * element count, rope_elems, right after the pointer, and returns
 * FAROPE_ERR_TABLE unless it equals farope_rope_packed_elems(n_pos,
 * head_dim / 2) of the call's descriptor.  (The reference never checks the
 * table against the attention shape, FA:1033, FA:1043-1047, and reads past
 * a short one.)
 */
#ifndef FAROPE_H
#define FAROPE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FAROPE_ABI_VERSION 5

typedef enum farope_dtype {
  FAROPE_F32 = 0,
  FAROPE_F16 = 1,
  FAROPE_BF16 = 2
} farope_dtype;

typedef enum farope_status {
  FAROPE_OK = 0,
  FAROPE_ERR_NULL = 1,        /* a required pointer is NULL */
  FAROPE_ERR_HEAD_DIM = 2,    /* head_dim not supported (needs D % 4 == 0; kernels: 32, 64, 128, 256) */
  FAROPE_ERR_SEQ_LEN = 3,     /* seq_len != n_pos + has_cls, or seq_len < 1 */
  FAROPE_ERR_DTYPE = 4,       /* unknown io or compute dtype */
  FAROPE_ERR_TABLE = 5,       /* rope_elems != farope_rope_packed_elems(n_pos, head_dim / 2),
                                 or farope_rope_pack given n_pos < 1 or an odd / zero d2 */
  FAROPE_ERR_SHAPE = 6,       /* batch/heads not positive or sizes overflow */
  FAROPE_ERR_LAUNCH = 7,      /* the HIP runtime rejected a kernel launch */
  FAROPE_ERR_ALIGN = 8,       /* a pointer is not aligned to its element size */
  FAROPE_ERR_SCRATCH = 9      /* workspace elems > FAROPE_NOALLOC_MAX_ROWS (noalloc entry) */
} farope_status;

/* Rows (batch * heads * seq_len) the static workspace of
 * farope_attn_bwd_noalloc holds: 4 Mi fp32 values = 16 MiB per device. */
#define FAROPE_NOALLOC_MAX_ROWS 4194304

/* Problem description shared by all attention entry points. */
typedef struct farope_attn_desc {
  int32_t batch;          /* B */
  int32_t heads;          /* H */
  int32_t seq_len;        /* N = n_pos + has_cls (FA:1016-1021) */
  int32_t head_dim;       /* D */
  int32_t n_pos;          /* rows of the RoPE grid, H_img * H_img */
  int32_t has_cls;        /* 1: token 0 is a CLS token and bypasses RoPE */
  int32_t io_dtype;       /* farope_dtype of q, k, v, o, dout, dq, dk, dv */
  int32_t compute_dtype;  /* farope_dtype the contractions run in (FA:65-73) */
  float softmax_scale;    /* 1/sqrt(D) in the reference (FA:1024) */
} farope_attn_desc;

/* ABI version of the loaded library (FAROPE_ABI_VERSION). */
int farope_abi_version(void);

/* Human-readable text for a farope_status code. */
const char* farope_strerror(int status);

/* Number of fp32 elements of a packed RoPE table: (n_pos + 1) * d2 * 2. */
size_t farope_rope_packed_elems(int32_t n_pos, int32_t d2);

/*
 * Re-lay the pairwise tables COSP/SINP [n_pos, d2] fp32 (any strides) into
 * the kernels' packed layout [(n_pos + 1), d2, (cos, sin)], row 0 = identity
 * rotation for the CLS token.  Replaces the per-tile transposed cos/sin
 * gathers of every reference kernel (FA:182-198, FA:253-269) with one
 * contiguous 32-byte load per 8 channels.  Tables built by
 * build_axial_rope_pairs (FA:10-63).
 */
int farope_rope_pack(const float* cosp, int64_t cos_stride0, int64_t cos_stride1,
                     const float* sinp, int64_t sin_stride0, int64_t sin_stride1,
                     int32_t n_pos, int32_t d2, float* packed, void* stream);

/*
 * Elements of the optional O residual buffer (o_res) a call uses:
 * batch * heads * seq_len * head_dim for bf16 tensors computed in bf16 at
 * head_dim >= 128, else 0.  Those calls take the logits, O = P V and the dQ /
 * dK products from fp16 operands; delta = rowsum(dout * o) taken from the
 * bf16-rounded o would then be the largest error term of dQ / dK, so the
 * forward can also store o's rounding residual bf16(o - bf16(o)) in a
 * contiguous [B, H, N, D] buffer of the I/O dtype, and the backward adds it
 * to o for delta.  No counterpart in the reference (whose delta uses the
 * stored o, FA:352-354).
 */
size_t farope_attn_residual_elems(const farope_attn_desc* desc);

/*
 * fp32 elements of farope_attn_bwd's delta_ws.  0 when the one-pass kernel
 * runs (head_dim 64, seq_len <= 256, 16-bit compute: it keeps delta on chip,
 * and delta_ws may then be NULL).  Otherwise batch * heads * seq_len delta
 * rows (the reference's D tensor, allocated with M's shape in
 * TritonAttention.backward, FA:1075), plus, when each plane's last key
 * is the only one past the dK/dV kernel's full key blocks at fp16-logit
 * shapes (bf16 compute, head_dim 128 or 256, N = 1 + a multiple of 256), one
 * partial dK / dV row pair per dQ tile: those tiles add that key's products
 * over their own query rows instead of a kernel that re-reads the plane;
 * then, at those fp16-logit shapes whenever every row lies in a dQ tile,
 * batch * heads * seq_len * head_dim fp16 values (from a 256-byte boundary):
 * the dQ pass's rotated Q rows, which the dK/dV pass stages instead of
 * rotating Q again for every key tile; then, of those shapes at head_dim
 * 128, 2 * batch * heads * seq_len fp32 values (from a 256-byte boundary):
 * each query row's {|dO|_2, max |Q-hat * scale * log2(e)|}, from which the
 * key-tile kernel fixes its fp16 operand scalings.  At the stored-dS shapes
 * (16-bit I/O, bf16 compute, head_dim 128, at most one key past the 128-key
 * tiles, and a dS^T plane of at most 16 Q planes: seq_len up to about 2k) the
 * larger of that and the stored-dS layout, whose parts each start
 * on a 256-byte boundary: the delta rows; with a lone last key one partial
 * dK / dV row pair per 64-row tile; the fp16 rotated Q rows; the row
 * statistics; with a lone last key its dS per query row; one int32 exponent
 * per key tile; the key tiles' fp16 K-hat rows; and their fp16 dS^T rows
 * (pitch seq_len rounded up to 64), which the dQ GEMM reads instead of
 * recomputing the logits.  0 on an invalid descriptor.
 */
size_t farope_attn_bwd_workspace_elems(const farope_attn_desc* desc);

/*
 * Forward: o = softmax(scale * (R q)(R k)^T) v, lse = logsumexp of the
 * scaled logits per row (natural log).  Replaces the _attn_fwd launch
 * (FA:1036-1057; kernel FA:91-315).  o_res: NULL, or a buffer of
 * farope_attn_residual_elems(desc) elements (filled when that is > 0).
 */
int farope_attn_fwd(const farope_attn_desc* desc,
                    const void* q, const int64_t q_stride[4],
                    const void* k, const int64_t k_stride[4],
                    const void* v, const int64_t v_stride[4],
                    const float* rope_packed, size_t rope_elems,
                    void* o, const int64_t o_stride[4], void* o_res,
                    float* lse, void* stream);

/* delta = rowsum(dout * (o + o_res)) in fp32 (o_res may be NULL).  Replaces
 * _attn_bwd_preprocess (launch FA:1076-1082; kernel FA:325-357). */
int farope_attn_bwd_preprocess(const farope_attn_desc* desc,
                               const void* o, const int64_t o_stride[4], const void* o_res,
                               const void* dout, const int64_t dout_stride[4],
                               float* delta, void* stream);

/* dk, dv from q, k, v, dout, lse, delta.  Replaces _attn_bwd_dk_dv_rope
 * (launch FA:1084-1107; kernel FA:374-691). */
int farope_attn_bwd_dk_dv(const farope_attn_desc* desc,
                          const void* q, const int64_t q_stride[4],
                          const void* k, const int64_t k_stride[4],
                          const void* v, const int64_t v_stride[4],
                          const void* dout, const int64_t dout_stride[4],
                          const float* lse, const float* delta,
                          const float* rope_packed, size_t rope_elems,
                          void* dk, const int64_t dk_stride[4],
                          void* dv, const int64_t dv_stride[4], void* stream);

/* dq from q, k, v, dout, lse, delta.  Replaces _attn_bwd_dq_rope
 * (launch FA:1109-1136; kernel FA:708-1009). */
int farope_attn_bwd_dq(const farope_attn_desc* desc,
                       const void* q, const int64_t q_stride[4],
                       const void* k, const int64_t k_stride[4],
                       const void* v, const int64_t v_stride[4],
                       const void* dout, const int64_t dout_stride[4],
                       const float* lse, const float* delta,
                       const float* rope_packed, size_t rope_elems,
                       void* dq, const int64_t dq_stride[4], void* stream);

/*
 * Whole backward pass (what TritonAttention.backward does, FA:1067-1138):
 * picks the fused one-launch kernel when the plane fits on chip (D = 64,
 * N <= 256); at the stored-dS shapes with vector access to every tensor a
 * row pass (delta), key tiles that keep dS, and dQ as one GEMM over it;
 * else dq (which also writes delta) followed by dk/dv.
 * delta_ws: caller-owned fp32 workspace of
 * farope_attn_bwd_workspace_elems(desc) elements.
 * o_res: NULL, or the residual buffer the forward filled.
 */
int farope_attn_bwd(const farope_attn_desc* desc,
                    const void* q, const int64_t q_stride[4],
                    const void* k, const int64_t k_stride[4],
                    const void* v, const int64_t v_stride[4],
                    const void* o, const int64_t o_stride[4], const void* o_res,
                    const void* dout, const int64_t dout_stride[4],
                    const float* lse, const float* rope_packed, size_t rope_elems,
                    void* dq, const int64_t dq_stride[4],
                    void* dk, const int64_t dk_stride[4],
                    void* dv, const int64_t dv_stride[4],
                    float* delta_ws, void* stream);

/*
 * farope_attn_bwd without the caller workspace: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  The split
 * path's workspace (the delta rows, and the partial rows of a lone last key)
 * lives in a static device array of FAROPE_NOALLOC_MAX_ROWS fp32 values that
 * the library holds on every device it runs on until the process ends; calls
 * that need more return FAROPE_ERR_SCRATCH before anything is launched.  The
 * rest of farope_attn_bwd_workspace_elems (rotated Q rows, row statistics,
 * the stored-dS planes) goes there too when the whole workspace fits, and the
 * kernels are then those of farope_attn_bwd; otherwise the split path's
 * kernels run, the generic dK/dV kernel rotating Q itself (results within
 * rounding of farope_attn_bwd's).  The one-pass
 * backward uses no workspace and takes any size.  Allocates nothing.  Calls
 * on one device share that array, so calls that overlap on one device
 * (concurrent streams or threads) race; calls ordered on one stream do not.
 * The current device must be the one holding the tensors.
 */
int farope_attn_bwd_noalloc(const farope_attn_desc* desc,
                            const void* q, const int64_t q_stride[4],
                            const void* k, const int64_t k_stride[4],
                            const void* v, const int64_t v_stride[4],
                            const void* o, const int64_t o_stride[4], const void* o_res,
                            const void* dout, const int64_t dout_stride[4],
                            const float* lse, const float* rope_packed, size_t rope_elems,
                            void* dq, const int64_t dq_stride[4],
                            void* dk, const int64_t dk_stride[4],
                            void* dv, const int64_t dv_stride[4], void* stream);

/*
 * Tile table query (replaces the reference's triton.autotune configs,
 * FA:76-90, FA:318-324, FA:359-373, FA:693-707).  which: 0 = forward,
 * 1 = backward.  out[0] = variant (fwd: 0 = persistent pipelined kernel,
 * 1 = one wave per (b, h) plane for 193 <= N <= 208 at head_dim 64 with
 * 16-bit tensors, assuming vector access; bwd: 0 fused, 1 split, 2 split with
 * the key-tile kernel, 3 key tiles that store dS and dQ as one GEMM over it,
 * assuming vector access), out[1] = query (fwd) or key (bwd) rows per work item,
 * out[2] = work items per (b, h) plane, out[3] = threads per workgroup.  When 1 to 8 rows are left past out[1] * out[2] (N = 1025 with
 * 128- or 256-row items), they are computed by the tail-row kernels (or, for
 * a single row with fp16 logit operands, by one designated item of each plane
 * in the forward and dQ block kernels) rather than by one more, nearly
 * empty, work item.
 */
int farope_tile_config(const farope_attn_desc* desc, int32_t which, int32_t out[4]);

#ifdef __cplusplus
}
#endif

#endif /* FAROPE_H */
