/*
 * cmpext3_attn.h -- C ABI of the MI355X (gfx950) fused attention forward.
 *
 * One entry point computes O = softmax(scale * Q K^T [+ causal mask]) V for
 * [B, H, S, D] tensors that already live in device memory.  The caller owns
 * every input and output buffer, and the library allocates no device memory
 * of its own.  Launches that split key ranges across workgroups (non-causal,
 * when the query blocks do not fill whole rounds of the GPU; fp16/bf16 with
 * D <= 128, fp16/bf16 with D > 128 and fewer query blocks than CUs, and fp32
 * with at most as many query blocks as CUs; causal fp16/bf16 grids that fill
 * at most half of the workgroup slots with long sweeps or on few CUs)
 * exchange partial results through
 * a caller-owned workspace (cmpext3_attn_fwd_ws, sized by
 * cmpext3_attn_fwd_workspace_size) or, in the allocation-free entry point,
 * through a fixed per-device array inside the library.  Every other call, and
 * any call whose workspace is null or too small, runs without the split (or
 * with fewer key ranges): the same result within rounding (a split adds the
 * parts' partial sums in another order, and two-part fp16 splits round each
 * part's O/l to fp16), bit-identical from one call to the next for a given
 * plan.  No launch ever waits for another workgroup, so no interleaving of
 * launches can hang the GPU.  All launches go on the stream the caller
 * passes.
 *
 * Reference interfaces this replaces (WifiLast/torch-cmp-patch):
 *   - launch_flash_attention_hfma2(q, k, v, o, B, H, Sq, Sk, D, qs, ks, vs, os,
 *     scale, stream) -> bool              src/cuda/fp16_flash_attention_hfma2.cu:269-272
 *   - launch_attention_fp16(q, k, v, o, B, H, S, D, scale, causal)
 *                                          src/main.cpp:93 (fp16_attention.cu:328-386)
 *   - launch_attention_fp32(q, k, v, o, B, H, S, D, scale)
 *                                          src/main.cpp:92 (fp32_attention.cu:200-221)
 * The three reference launchers are merged into one call that takes the
 * dtype as an argument, accepts Sq != Sk and causal masking for every dtype,
 * and reports failure through a return code instead of silently returning
 * (the reference's fp16/fp32 launchers return void and may leave the output
 * unwritten, src/main.cpp:1741-1765).
 *
 * Strides are in ELEMENTS, ordered {batch, head, seq}; the last (head-dim)
 * dimension must be contiguous, as in the reference's HFMA2 launcher.
 */
#ifndef CMPEXT3_ATTN_H
#define CMPEXT3_ATTN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CMPEXT3_ATTN_ABI_VERSION 9

/* dtype codes (CMPEXT3_DTYPE_BOOL: attention masks only) */
#define CMPEXT3_DTYPE_F16  0
#define CMPEXT3_DTYPE_BF16 1
#define CMPEXT3_DTYPE_F32  2
#define CMPEXT3_DTYPE_BOOL 3

/* workspace layout: counters first (cmpext3_attn_fwd_ws), and the size of
   the allocation-free entry point's fixed per-device array */
#define CMPEXT3_WORKSPACE_COUNTER_BYTES 65536
#define CMPEXT3_NOALLOC_SCRATCH_BYTES (65536 + 16777216)

/* return codes */
#define CMPEXT3_OK                 0
#define CMPEXT3_E_INVALID          1  /* null pointer, negative size, bad stride */
#define CMPEXT3_E_DTYPE            2  /* dtype code not one of the above */
#define CMPEXT3_E_HEAD_DIM         3  /* D outside 1..256; training calls: D not a multiple of 8 (f16/bf16); masked calls: D odd (f16/bf16) or not a multiple of 4 (f32) */
#define CMPEXT3_E_ALIGN            4  /* a pointer not element-aligned; training and fp32 masked calls: base pointer or row stride not 16-byte aligned; f16/bf16 masked calls: not 4-byte aligned */
#define CMPEXT3_E_EMPTY_KEYS       5  /* Sk == 0 with Sq > 0: softmax over nothing */
#define CMPEXT3_E_LAUNCH           6  /* the HIP launch itself failed */
#define CMPEXT3_E_TOO_LARGE        7  /* a size does not fit the kernel's index arithmetic */
#define CMPEXT3_E_MASK             8  /* attention mask the library cannot take (none at present) */
#define CMPEXT3_E_TRAINING         9  /* training call the library cannot take (none at present) */

/*
 * Fused attention forward.
 *
 *   q : [B, H, Sq, D]   k, v : [B, H, Sk, D]   o : [B, H, Sq, D]  (all `dtype`)
 *   *_str[3] : element strides of dims {0, 1, 2} (>= 0); dim 3 has stride 1.
 *   D        : any head dim 1..256.  Pointers need only element alignment:
 *              rows of whole 16-byte chunks with 16-byte aligned base
 *              pointers and strides run the vector-load kernels; any other
 *              layout (odd D, a 2-byte offset view, BSHD views of such
 *              heads) runs element-granular variants of the same kernels in
 *              place, with no copy (calls that pass a mask, and the
 *              training entry points, still need whole 16-byte aligned
 *              chunks: CMPEXT3_E_HEAD_DIM / CMPEXT3_E_ALIGN otherwise).
 *   scale    : multiplier of Q K^T (any finite value, 0 and negative allowed).
 *   causal   : non-zero -> key j is visible to query i iff j <= i
 *              (top-left aligned, the torch `is_causal` convention also for
 *              Sq != Sk).
 *   stream   : HIP stream to launch on (0 = the null stream).
 *
 * Returns CMPEXT3_OK, or one of the CMPEXT3_E_* codes above, in which case
 * nothing was launched except for CMPEXT3_E_LAUNCH.  B*H*Sq == 0 is a no-op.
 * Thread-safe; no host synchronisation; nothing is allocated: this entry
 * point never splits key ranges (cmpext3_attn_fwd_ws with a workspace does).
 */
int cmpext3_attn_fwd(const void* q, const void* k, const void* v, void* o,
                     int dtype, int B, int H, int Sq, int Sk, int D,
                     const int64_t q_str[3], const int64_t k_str[3],
                     const int64_t v_str[3], const int64_t o_str[3],
                     float scale, int causal, hipStream_t stream);

/*
 * Grouped-query attention: as cmpext3_attn_fwd, with k and v holding H_kv
 * heads ([B, H_kv, Sk, D]) shared by groups of H / H_kv consecutive query
 * heads (query head h reads K/V head h / (H / H_kv)), the torch
 * scaled_dot_product_attention(..., enable_gqa=True) semantics.  H_kv must
 * divide H (else CMPEXT3_E_INVALID); H_kv == H is cmpext3_attn_fwd.
 *
 * Reference: the reference's patch hands enable_gqa only to stock torch
 * (cmpext3/__init__.py:632-633) and its kernels require equal head counts
 * (src/main.cpp:1603-1774), so GQA calls always left the native path; this
 * entry point keeps them on it without repeating K/V per query head.
 */
int cmpext3_attn_fwd_gqa(const void* q, const void* k, const void* v, void* o,
                         int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                         const int64_t q_str[3], const int64_t k_str[3],
                         const int64_t v_str[3], const int64_t o_str[3],
                         float scale, int causal, hipStream_t stream);

/*
 * Attention with an explicit mask: as cmpext3_attn_fwd_gqa, plus torch's
 * scaled_dot_product_attention attn_mask.
 *
 *   mask       : device pointer, aligned to its element size.
 *   mask_dtype : CMPEXT3_DTYPE_BOOL (one byte per element; non-zero keeps the
 *                (query, key) pair, zero drops it) or CMPEXT3_DTYPE_F16 /
 *                _BF16 / _F32 (added to scale * Q K^T, -inf drops the pair);
 *                -1 means no mask (then mask and mask_str are ignored).
 *   mask_str[3]: element strides of the mask over {batch, head, query}
 *                (0 = broadcast, otherwise any non-negative value); keys are
 *                contiguous (stride 1).  Element (b, h, i, j) lives at
 *                mask + b*mask_str[0] + h*mask_str[1] + i*mask_str[2] + j.
 *                Nothing past key Sk - 1 of a row is read.  (With a 16-byte
 *                aligned mask, strides that are multiples of 4 and Sk a
 *                multiple of 8 the keys are read in runs of 8; any other
 *                layout element by element.)
 * A query row whose keys are all dropped gives zeros (torch's result).
 * With causal != 0 a pair is used only if it is causally visible AND the
 * mask keeps it (torch's rule for attn_mask with is_causal).  Supported for
 * every dtype (f16, bf16, f32) and head dim; the rows of q/k/v/o must be
 * whole 16-byte chunks at 16-byte aligned addresses for f32, and 4-byte
 * aligned (even D, base pointers and row strides) for f16/bf16 (else
 * CMPEXT3_E_ALIGN or CMPEXT3_E_HEAD_DIM, nothing launched).
 *
 * Reference: the reference never ran masks natively: _patched_sdpa sends
 * any attn_mask to stock torch (cmpext3/__init__.py:624).
 */
int cmpext3_attn_fwd_masked(const void* q, const void* k, const void* v, void* o,
                            int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                            const int64_t q_str[3], const int64_t k_str[3],
                            const int64_t v_str[3], const int64_t o_str[3],
                            const void* mask, int mask_dtype, const int64_t mask_str[3],
                            float scale, int causal, hipStream_t stream);

/*
 * Workspace forward: the arguments, results and return codes of
 * cmpext3_attn_fwd_masked (mask_dtype -1 = no mask, H_kv == H = no
 * grouping), plus a caller-owned device workspace for the key split.
 *
 *   workspace       : device memory, 16-byte aligned (else CMPEXT3_E_ALIGN),
 *                     or null (no split).
 *   workspace_bytes : its size.  cmpext3_attn_fwd_workspace_size gives the
 *                     bytes the full split plan of a problem takes; with
 *                     less, the launch cuts its blocks into fewer key ranges,
 *                     or runs unsplit.  Nothing is ever refused for it.
 * The workspace's first CMPEXT3_WORKSPACE_COUNTER_BYTES (64 KiB) are
 * counters: they must be zero before the
 * workspace is first used, and every launch leaves them zero when it
 * completes, so one workspace can serve any sequence of calls, of any
 * shapes, that run one after another (for example every call on one
 * stream).  The rest needs no initialisation.  Two launches that may run at
 * the same time must not share a workspace: they would not hang, but they
 * could mix each other's partial results (wrong output, counters left
 * non-zero for later calls).  The workspace is only read and written by the
 * launch's kernels on `stream`.
 *
 * Reference: launch_flash_attention_hfma2 (src/cuda/fp16_flash_attention_hfma2.cu:269-272)
 * takes no workspace; it never splits a block's keys.
 */
int cmpext3_attn_fwd_ws(const void* q, const void* k, const void* v, void* o,
                        int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                        const int64_t q_str[3], const int64_t k_str[3],
                        const int64_t v_str[3], const int64_t o_str[3],
                        const void* mask, int mask_dtype, const int64_t mask_str[3],
                        float scale, int causal, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/*
 * Workspace bytes cmpext3_attn_fwd_ws (with_lse 0) or cmpext3_attn_fwd_lse
 * (with_lse 1) needs to run the full key-split plan of this problem, for any
 * row layout of its tensors; 0 when the problem never splits or the
 * arguments are invalid.  Depends on the device's CU count (the current
 * device; 256, MI355X's, when none is visible).  Host-only.
 */
size_t cmpext3_attn_fwd_workspace_size(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                                       int mask_dtype, int causal, int with_lse);

/*
 * The key split a launch of this problem (contiguous [B,H,S,D] tensors) takes
 * with workspace_bytes of workspace: *key_parts receives the key ranges each
 * split query block is cut into (1 = unsplit; 0 on error).  Returns the code
 * the launch would return before launching.  Host-only: runs the launch's
 * own dispatch up to the point of launching.
 */
int cmpext3_attn_fwd_plan(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D, int mask_dtype,
                          int causal, int with_lse, size_t workspace_bytes, int* key_parts);

/*
 * Allocation-free forward: the arguments, results and return codes of
 * cmpext3_attn_fwd_masked (mask_dtype -1 = no mask, H_kv == H = no grouping),
 * but nothing is ever allocated or freed: key-split launches exchange their
 * partial results through a fixed array of CMPEXT3_NOALLOC_SCRATCH_BYTES
 * (64 KiB of counters + 16 MiB) per device inside the library's code
 * object: every call behaves as cmpext3_attn_fwd_ws with a workspace of
 * that size (same plan, same result bit for bit).  A split that would need more is cut to
 * fewer key ranges (down to none), so no problem is refused for lack of
 * room.  Every call on one device shares that device's array: calls in
 * stream order are safe; calls that overlap in time on one device (two
 * streams, or a graph replay beside an eager call) must not be made -- they
 * cannot hang (no launch waits for another workgroup), but they can give
 * wrong results and leave counters non-zero, which can make later split
 * calls on that device wrong too.  Launches may be captured into a HIP graph
 * (the array's address is fixed).
 *
 * Reference: none.  No counterpart in the reference; it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * with a fixed memory budget, harnesses that forbid hipMalloc).
 */
int cmpext3_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* o,
                             int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                             const int64_t q_str[3], const int64_t k_str[3],
                             const int64_t v_str[3], const int64_t o_str[3],
                             const void* mask, int mask_dtype, const int64_t mask_str[3],
                             float scale, int causal, hipStream_t stream);

/*
 * Training forward: as cmpext3_attn_fwd_masked (mask_dtype -1 = no mask), and
 * also writes
 *
 *   lse : [B, H, Sq] fp32, contiguous (element (b, h, i) at lse[(b*H + h)*Sq + i]),
 *         the natural-log log-sum-exp over the visible keys of row i of
 *         scale * Q K^T (+ mask) -- what cmpext3_attn_bwd needs to rebuild the
 *         softmax; -inf for a row whose keys are all dropped.
 *
 * Every dtype (rows in whole, 16-byte aligned chunks, else CMPEXT3_E_ALIGN /
 * CMPEXT3_E_HEAD_DIM).  f16/bf16 calls run the pipelined kernel up to
 * D = 128, whatever Sk, and above it (192 and 256 buckets) when Sq > 64 and
 * Sk >= 256 (both may key-split through the workspace); other f16/bf16
 * calls above D = 128 run the head-dim > 128 kernel (never key-split here),
 * and fp32 calls the fp32 kernel (key-split like its inference launch).  A mask
 * is read in runs of 8 keys, as the backward reads it: 16-byte aligned,
 * strides multiples of 4 elements (else CMPEXT3_E_ALIGN), and every row
 * readable up to Sk rounded up to a multiple of 8 (values past Sk are
 * ignored).
 * workspace / workspace_bytes: as in cmpext3_attn_fwd_ws (null: no split;
 * size from cmpext3_attn_fwd_workspace_size with with_lse = 1).
 *
 * Reference: none.  The reference is forward-only: its patch hands every
 * call with live autograd to stock torch (cmpext3/__init__.py:115-125).
 */
int cmpext3_attn_fwd_lse(const void* q, const void* k, const void* v, void* o, float* lse,
                         int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                         const int64_t q_str[3], const int64_t k_str[3],
                         const int64_t v_str[3], const int64_t o_str[3],
                         const void* mask, int mask_dtype, const int64_t mask_str[3],
                         float scale, int causal, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

/*
 * Backward of the attention above: given q, k, v, the forward output o, its
 * gradient dout and the forward's lse, writes the gradients
 *
 *   dq : [B, H, Sq, D]   dk, dv : [B, H_kv, Sk, D]   (all `dtype`, overwritten)
 *
 * of sum(o * dout), with the same scale, causal flag, K/V head count and
 * attention mask (the layout rules of cmpext3_attn_fwd_lse; -1 = none) as
 * the forward (H_kv must divide H; query head h uses K/V head h / (H / H_kv),
 * and dk, dv sum the contributions of every query head of the group).  A row
 * whose keys were all dropped passes no gradient (its dq row is zero).
 *   delta : caller-owned fp32 workspace of B*H*Sq elements (4-byte aligned;
 *           receives sum_d dout * o per row).
 *   *_str[3] : element strides over {batch, head, seq} as in cmpext3_attn_fwd.
 * Three kernels on `stream`: Delta, dK/dV (one workgroup per 128 keys of a
 * K/V head; 64 for fp32), dQ (one per 128 queries; 64 for fp32); each
 * gradient row is written by exactly one workgroup, so results are
 * bit-identical from run to run.  This entry point takes no workspace and
 * never splits a sweep (cmpext3_attn_bwd_ws below can).  B*H*Sq == 0 is a no-op (dk and dv are then
 * left untouched).  Every dtype: f16/bf16 on 32x32x16 MFMAs (head dims above
 * 128 in the 192 and 256 buckets at one wave per SIMD), fp32 on 16x16x4 fp32
 * MFMAs (buckets 32, 40, 64, 96, 128, 192, 256).
 *
 * Reference: none (forward-only reference, cmpext3/__init__.py:115-125).
 */
int cmpext3_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                     const void* dout, const float* lse, void* dq, void* dk, void* dv,
                     float* delta, int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                     const int64_t q_str[3], const int64_t k_str[3],
                     const int64_t v_str[3], const int64_t o_str[3],
                     const int64_t do_str[3], const int64_t dq_str[3],
                     const int64_t dk_str[3], const int64_t dv_str[3],
                     const void* mask, int mask_dtype, const int64_t mask_str[3],
                     float scale, int causal, hipStream_t stream);

/*
 * cmpext3_attn_bwd with a caller-owned workspace (16-byte aligned; NULL or 0
 * bytes = none).  Problems with too few key blocks for the CUs
 * (grouped-query K/V of one or two sequences, causal sweeps whose length
 * falls with the key block) cut each block's dK/dV sweep over (query head,
 * query tile) into up to 8 contiguous parts on separate workgroups, and
 * likewise the dQ sweeps of few query blocks over key tiles (f16/bf16
 * non-causal grids past one round split only their last, partial round of
 * blocks); the parts leave
 * fp32 partial rows in the workspace that a further kernel sums in part
 * order (still bit-identical from run to run; the sums differ from the
 * unsplit launch's only by rounding).  With a workspace smaller than
 * cmpext3_attn_bwd_workspace_size, a sweep whose partials do not fit runs
 * unsplit (the dK/dV partials take the workspace first).  Otherwise the arguments,
 * results and return codes of cmpext3_attn_bwd (CMPEXT3_E_ALIGN also for a
 * misaligned workspace).
 *
 * Reference: none (forward-only reference, cmpext3/__init__.py:115-125).
 */
int cmpext3_attn_bwd_ws(const void* q, const void* k, const void* v, const void* o,
                        const void* dout, const float* lse, void* dq, void* dk, void* dv,
                        float* delta, int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                        const int64_t q_str[3], const int64_t k_str[3],
                        const int64_t v_str[3], const int64_t o_str[3],
                        const int64_t do_str[3], const int64_t dq_str[3],
                        const int64_t dk_str[3], const int64_t dv_str[3],
                        const void* mask, int mask_dtype, const int64_t mask_str[3],
                        float scale, int causal, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/*
 * Workspace bytes cmpext3_attn_bwd_ws needs to split this problem's gradient
 * sweeps (mask_dtype -1 = no mask); 0 when it never splits (enough blocks)
 * or the arguments are invalid.  Depends on the current device's CU
 * count (256, MI355X's, when none is visible).  Host-only.
 */
size_t cmpext3_attn_bwd_workspace_size(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                                       int mask_dtype, int causal);

/* Human-readable text for a return code (static storage). */
const char* cmpext3_attn_strerror(int code);

/* CMPEXT3_ATTN_ABI_VERSION of the loaded library. */
int cmpext3_attn_abi_version(void);

/*
 * Which kernel family and tile shape cmpext3_attn_fwd would pick for these
 * arguments, written as text into buf (at most len bytes, NUL-terminated).
 * Returns the same code cmpext3_attn_fwd would return before launching.
 * Host-only: touches no device.
 */
int cmpext3_attn_describe(int dtype, int B, int H, int Sq, int Sk, int D,
                          int causal, char* buf, int len);

#ifdef __cplusplus
}
#endif

#endif /* CMPEXT3_ATTN_H */
