// C ABI of the fused attention forward: argument validation and kernel dispatch.
//
// Replaces the reference's three launchers (launch_flash_attention_hfma2,
// launch_attention_fp16, launch_attention_fp32; src/main.cpp:92-108) and the
// shape/alignment checks its torch binding does before calling them
// (src/main.cpp:1637-1650, 1669-1681, 1741-1768).  Unsupported input is
// reported by return code and nothing is launched, so the caller can fall
// back; the reference's void launchers instead skipped the launch and left the
// output unwritten (src/main.cpp:1741-1765).
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/cmpext3_attn.h"
#include "attn_common.h"

#include "attn_bwd16.h"

namespace cmpext3 {
hipError_t launch_bwd16(const BwdParams& p, bool bf16, bool causal, hipStream_t s);
BwdSplit bwd16_split(int B, int H, int Hkv, int Sq, int Sk, int D, bool causal, bool masked, int cus);
BwdSplit bwd32_split(int B, int H, int Hkv, int Sq, int Sk, int D, bool causal, int cus);
// Split plan of the backward's gradient sweeps.
BwdSplit bwd_split(int dtype, int B, int H, int Hkv, int Sq, int Sk, int D, bool causal, bool masked) {
  return dtype == CMPEXT3_DTYPE_F32 ? bwd32_split(B, H, Hkv, Sq, Sk, D, causal, device_cus())
                                    : bwd16_split(B, H, Hkv, Sq, Sk, D, causal, masked, device_cus());
}
hipError_t launch_bwd32(const BwdParams& p, bool causal, hipStream_t s);
hipError_t launch_mfma16(const FwdParams& p, bool bf16, bool causal, hipStream_t s);
hipError_t launch_mfma32(const FwdParams& p, bool causal, hipStream_t s);
int mfma16_bucket(int D);
int mfma32_bucket(int D);
void describe_mfma16(int D, int B, int H, int Sq, int Sk, bool causal, bool bf16, char* buf, int len);
void describe_mfma32(int D, int B, int H, int Sq, int Sk, bool causal, char* buf, int len);
}  // namespace cmpext3

namespace {

int elem_size(int dtype) {
  switch (dtype) {
    case CMPEXT3_DTYPE_F16:
    case CMPEXT3_DTYPE_BF16: return 2;
    case CMPEXT3_DTYPE_F32: return 4;
  }
  return 0;
}

// Checks that need no pointers: sizes, dtype, head dim.
int check_shape(int dtype, int B, int H, int Sq, int Sk, int D) {
  const int es = elem_size(dtype);
  if (es == 0) return CMPEXT3_E_DTYPE;
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0 || D < 0) return CMPEXT3_E_INVALID;
  if ((int64_t)B * H * Sq == 0) return CMPEXT3_OK;  // nothing to compute
  if (Sk == 0) return CMPEXT3_E_EMPTY_KEYS;
  if (D == 0 || D > 256) return CMPEXT3_E_HEAD_DIM;
  // workgroup count and in-kernel int arithmetic on (b*H + h) and row indices
  if ((int64_t)B * H * ((Sq + 63) / 64) > (int64_t)INT32_MAX / 2) return CMPEXT3_E_TOO_LARGE;
  if (Sq > INT32_MAX - 512 || Sk > INT32_MAX - 512) return CMPEXT3_E_TOO_LARGE;
  return CMPEXT3_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }
bool aligned_to(const void* ptr, int es) { return ((uintptr_t)ptr % (uintptr_t)es) == 0; }
// rows of whole 16-byte chunks (the pipelined, short-key and training kernels)
bool whole_chunks(int dtype, int D) { return D % (16 / elem_size(dtype)) == 0; }

// attention-mask arguments (mask_dtype -1 = none): CMPEXT3_OK or an error code.
// Every dtype and head dim takes a mask (causal or not; the rows of Q, K, V
// and O must then be whole aligned 16-byte chunks, checked by the caller).
// The kernels read a mask in runs of 8 keys when its base is 16-byte aligned
// and its strides are multiples of 4 elements (*runs_ok); the inference entry
// points read any other element-aligned layout element by element.
int check_mask(const void* mask, int mask_dtype, const int64_t mask_str[3], int Sq, int Sk, bool* runs_ok) {
  *runs_ok = true;
  if (mask_dtype == -1) return CMPEXT3_OK;
  if (mask_dtype < CMPEXT3_DTYPE_F16 || mask_dtype > CMPEXT3_DTYPE_BOOL) return CMPEXT3_E_DTYPE;
  if (!mask || !mask_str) return CMPEXT3_E_INVALID;
  const int mes = mask_dtype == CMPEXT3_DTYPE_BOOL ? 1 : mask_dtype == CMPEXT3_DTYPE_F32 ? 4 : 2;
  if (((uintptr_t)mask % (uintptr_t)mes) != 0) return CMPEXT3_E_ALIGN;
  for (int i = 0; i < 3; ++i)
    if (mask_str[i] < 0) return CMPEXT3_E_ALIGN;
  *runs_ok = ((uintptr_t)mask & 15u) == 0 && mask_str[0] % 4 == 0 && mask_str[1] % 4 == 0 && mask_str[2] % 4 == 0;
  if (((int64_t)(Sq - 1) * mask_str[2] + Sk + 64) * mes >= INT32_MAX) return CMPEXT3_E_TOO_LARGE;
  return CMPEXT3_OK;
}

int mask_kind_of(int mask_dtype) {
  return mask_dtype == CMPEXT3_DTYPE_BOOL ? cmpext3::MASK_BOOL
         : mask_dtype == CMPEXT3_DTYPE_F32 ? cmpext3::MASK_F32
         : mask_dtype == CMPEXT3_DTYPE_BF16 ? cmpext3::MASK_BF16 : cmpext3::MASK_F16;
}

// A stride only matters if its dimension has more than one index: each must
// be non-negative and a multiple of 16 bytes (es = element size).
bool stride_ok(const int64_t s[3], int n0, int n1, int n2, int es) {
  const int64_t n[3] = {n0, n1, n2};
  for (int i = 0; i < 3; ++i) {
    if (n[i] <= 1) continue;
    if (s[i] < 0) return false;
    if ((s[i] * es) % 16 != 0) return false;
  }
  return true;
}
// Largest of 2, 4, 8, 16 bytes dividing every base pointer, every row stride
// (of a dimension with more than one index) and the row length D * es.
int piece_bytes(const void* q, const void* k, const void* v, const void* o, int D, int es,
                const int64_t q_str[3], const int64_t k_str[3], const int64_t v_str[3],
                const int64_t o_str[3], int B, int H, int H_kv, int Sq, int Sk) {
  uint64_t bits = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)o | (uint64_t)D * es;
  auto add = [&](const int64_t s[3], int n0, int n1, int n2) {
    const int64_t n[3] = {n0, n1, n2};
    for (int i = 0; i < 3; ++i)
      if (n[i] > 1) bits |= (uint64_t)s[i] * es;
  };
  add(q_str, B, H, Sq);
  add(k_str, B, H_kv, Sk);
  add(v_str, B, H_kv, Sk);
  add(o_str, B, H, Sq);
  return (bits & 15) == 0 ? 16 : (bits & 7) == 0 ? 8 : (bits & 3) == 0 ? 4 : 2;
}

bool strides_nonneg(const int64_t s[3], int n0, int n1, int n2) {
  const int64_t n[3] = {n0, n1, n2};
  for (int i = 0; i < 3; ++i)
    if (n[i] > 1 && s[i] < 0) return false;
  return true;
}

}  // namespace

extern "C" {

int cmpext3_attn_abi_version(void) { return CMPEXT3_ATTN_ABI_VERSION; }

const char* cmpext3_attn_strerror(int code) {
  switch (code) {
    case CMPEXT3_OK: return "success";
    case CMPEXT3_E_INVALID: return "invalid argument (null pointer, negative size or stride)";
    case CMPEXT3_E_DTYPE: return "unsupported dtype (expected f16, bf16 or f32)";
    case CMPEXT3_E_HEAD_DIM:
      return "unsupported head dim (need 1..256; training calls and fp32 masked calls need a multiple of 8 for "
             "f16/bf16, 4 for f32; f16/bf16 masked calls an even head dim)";
    case CMPEXT3_E_ALIGN:
      return "misaligned tensor (pointers must be element-aligned; training calls and fp32 masked calls need "
             "16-byte aligned base pointers and row strides, f16/bf16 masked calls 4-byte aligned ones)";
    case CMPEXT3_E_EMPTY_KEYS: return "key/value sequence is empty";
    case CMPEXT3_E_LAUNCH: return "HIP kernel launch failed";
    case CMPEXT3_E_TOO_LARGE: return "problem too large for 32-bit tile indexing";
    case CMPEXT3_E_MASK:
      return "attention mask not supported here";
    case CMPEXT3_E_TRAINING:
      return "not supported by the training entry points (none at present)";
  }
  return "unknown error code";
}

int cmpext3_attn_describe(int dtype, int B, int H, int Sq, int Sk, int D, int causal, char* buf,
                          int len) {
  const int rc = check_shape(dtype, B, H, Sq, Sk, D);
  if (buf && len > 0) {
    if (rc != CMPEXT3_OK) {
      snprintf(buf, len, "unsupported: %s", cmpext3_attn_strerror(rc));
    } else if ((int64_t)B * H * Sq == 0) {
      snprintf(buf, len, "empty problem: no launch");
    } else {
      char kb[320];
      if (dtype == CMPEXT3_DTYPE_F32)
        cmpext3::describe_mfma32(D, B, H, Sq, Sk, causal != 0, kb, sizeof kb);
      else
        cmpext3::describe_mfma16(D, B, H, Sq, Sk, causal != 0, dtype == CMPEXT3_DTYPE_BF16, kb, sizeof kb);
      snprintf(buf, len, "%s%s", kb, causal ? " causal" : "");
    }
  }
  return rc;
}

int cmpext3_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H,
                     int Sq, int Sk, int D, const int64_t q_str[3], const int64_t k_str[3],
                     const int64_t v_str[3], const int64_t o_str[3], float scale, int causal,
                     hipStream_t stream) {
  return cmpext3_attn_fwd_gqa(q, k, v, o, dtype, B, H, H, Sq, Sk, D, q_str, k_str, v_str, o_str, scale,
                              causal, stream);
}

int cmpext3_attn_fwd_gqa(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                         int H, int H_kv, int Sq, int Sk, int D, const int64_t q_str[3],
                         const int64_t k_str[3], const int64_t v_str[3], const int64_t o_str[3],
                         float scale, int causal, hipStream_t stream) {
  return cmpext3_attn_fwd_masked(q, k, v, o, dtype, B, H, H_kv, Sq, Sk, D, q_str, k_str, v_str, o_str,
                                 nullptr, -1, nullptr, scale, causal, stream);
}

}  // extern "C"

namespace {

// Byte offsets of every row of an S-row sweep, plus one 64-row tile past it,
// stay below 2^31 (the pipelined and backward kernels' 32-bit buffer offsets)
// for es-byte elements.
bool tile_offsets_fit(int S, int64_t s0, int64_t s1, int es = 2) {
  const int64_t rs = s0 > s1 ? s0 : s1;
  return (int64_t)(S + 64) * rs * es < INT32_MAX;
}

// Forward with every option; lse (may be null) receives the row log-sum-exp.
int fwd_impl(const void* q, const void* k, const void* v, void* o, float* lse, int dtype, int B, int H,
             int H_kv, int Sq, int Sk, int D, const int64_t q_str[3], const int64_t k_str[3],
             const int64_t v_str[3], const int64_t o_str[3], const void* mask, int mask_dtype,
             const int64_t mask_str[3], float scale, int causal, hipStream_t stream,
             void* workspace, size_t workspace_bytes, bool fixed_exchange = false) {
  int rc = check_shape(dtype, B, H, Sq, Sk, D);
  if (rc != CMPEXT3_OK) return rc;
  if ((int64_t)B * H * Sq == 0) return CMPEXT3_OK;
  if (H_kv < 1 || H_kv > H || H % H_kv != 0) return CMPEXT3_E_INVALID;
  const bool masked = mask_dtype != -1;
  bool runs_ok = true;
  rc = check_mask(mask, mask_dtype, mask_str, Sq, Sk, &runs_ok);
  if (rc != CMPEXT3_OK) return rc;
  // The training forward's mask is the backward's too: runs of 8 keys, rows
  // readable up to Sk rounded up to 8 (the caller pads them).  Inference
  // calls read runs only where every row ends on a whole run.
  if (lse && !runs_ok) return CMPEXT3_E_ALIGN;
  const bool narrow_mask = !lse && (!runs_ok || Sk % 8 != 0);
  if (!q || !k || !v || !o || !q_str || !k_str || !v_str || !o_str) return CMPEXT3_E_INVALID;
  if (!isfinite(scale)) return CMPEXT3_E_INVALID;
  if (workspace && !aligned16(workspace)) return CMPEXT3_E_ALIGN;
  const int es = elem_size(dtype);
  if (!aligned_to(q, es) || !aligned_to(k, es) || !aligned_to(v, es) || !aligned_to(o, es))
    return CMPEXT3_E_ALIGN;
  if (!strides_nonneg(q_str, B, H, Sq) || !strides_nonneg(k_str, B, H_kv, Sk) ||
      !strides_nonneg(v_str, B, H_kv, Sk) || !strides_nonneg(o_str, B, H, Sq))
    return CMPEXT3_E_INVALID;
  // Rows of whole, 16-byte aligned chunks run the vector-load kernels; any
  // other layout (head dim not a multiple of 16 bytes, a base pointer or row
  // stride off 16 bytes) runs the narrow variants in place, in pieces of the
  // largest of 2, 4, 8 bytes that divides every address, row stride and the
  // row length.  Those exist for unmasked inference only.
  const int piece = piece_bytes(q, k, v, o, D, es, q_str, k_str, v_str, o_str, B, H, H_kv, Sq, Sk);
  const bool chunks = piece == 16;
  // Training calls need whole aligned chunks; masked ones also run on 4- or
  // 8-byte pieces of f16/bf16 rows (fp32 and 2-byte pieces: whole chunks).
  const bool mask_rows_ok = !masked || chunks || (dtype != CMPEXT3_DTYPE_F32 && piece >= 4);
  if ((!chunks && lse) || !mask_rows_ok) return whole_chunks(dtype, D) ? CMPEXT3_E_ALIGN : CMPEXT3_E_HEAD_DIM;
  // the fp16/bf16 kernel addresses one K/V tile with 32-bit element offsets
  if (dtype != CMPEXT3_DTYPE_F32 &&
      (k_str[2] * 64 + 256 > INT32_MAX || v_str[2] * 64 + 256 > INT32_MAX))
    return CMPEXT3_E_TOO_LARGE;
  // the pipelined kernel (every masked or training call up to D = 128) and
  // the backward address every K/V tile of the sweep with 32-bit buffer
  // offsets; masked and training calls keep that one limit at every head dim
  if ((masked || lse) && !tile_offsets_fit(Sk, k_str[2], v_str[2], es)) return CMPEXT3_E_TOO_LARGE;

  cmpext3::FwdParams p;
  memset(&p, 0, sizeof p);
  p.q = q; p.k = k; p.v = v; p.o = o;
  p.q_b = q_str[0]; p.q_h = q_str[1]; p.q_s = q_str[2];
  p.k_b = k_str[0]; p.k_h = k_str[1]; p.k_s = k_str[2];
  p.v_b = v_str[0]; p.v_h = v_str[1]; p.v_s = v_str[2];
  p.o_b = o_str[0]; p.o_h = o_str[1]; p.o_s = o_str[2];
  p.B = B; p.H = H; p.Sq = Sq; p.Sk = Sk; p.D = D;
  p.kv_group = H / H_kv;  // query head h reads K/V head h / kv_group
  p.mask_kind = cmpext3::MASK_NONE;
  p.lse = lse;
  if (masked) {
    p.mask = mask;
    p.m_b = mask_str[0]; p.m_h = mask_str[1]; p.m_q = mask_str[2];
    p.mask_kind = mask_kind_of(mask_dtype);
    p.mask_narrow = narrow_mask ? 1 : 0;
  }
  // exp2-domain multiplier; a negative scale is folded into Q's sign bits
  p.c = fabsf(scale) * cmpext3::kLog2e;
  p.q_sign = (scale < 0.f) ? (dtype == CMPEXT3_DTYPE_F32 ? 0x80000000u : 0x80008000u) : 0u;
  p.fixed_exchange = fixed_exchange ? 1 : 0;
  p.workspace = workspace;
  p.workspace_bytes = workspace ? workspace_bytes : 0;
  p.elem_rows = chunks ? 0 : piece;

  hipError_t err;
  if (dtype == CMPEXT3_DTYPE_F32)
    err = cmpext3::launch_mfma32(p, causal != 0, stream);
  else
    err = cmpext3::launch_mfma16(p, dtype == CMPEXT3_DTYPE_BF16, causal != 0, stream);
  return err == hipSuccess ? CMPEXT3_OK : CMPEXT3_E_LAUNCH;
}

// Dry run of the forward dispatch for a problem in contiguous [B,H,S,D]
// layout whose rows are read in `elem`-byte pieces (0: whole 16-byte
// chunks): the same launchers as fwd_impl with FwdParams::dry set, so the
// plan recorded is the one a launch would take with workspace_bytes of
// workspace.  Touches no device (the CU count falls back to MI355X's 256
// when none is visible).
int plan_impl(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D, int mask_dtype, int causal,
              int with_lse, int elem, size_t workspace_bytes, cmpext3::SplitInfo& info) {
  info.need = 0;
  info.parts = 1;
  int rc = check_shape(dtype, B, H, Sq, Sk, D);
  if (rc != CMPEXT3_OK || (int64_t)B * H * Sq == 0) return rc;
  if (H_kv < 1 || H_kv > H || H % H_kv != 0) return CMPEXT3_E_INVALID;
  if (mask_dtype != -1 && (mask_dtype < CMPEXT3_DTYPE_F16 || mask_dtype > CMPEXT3_DTYPE_BOOL))
    return CMPEXT3_E_DTYPE;
  if (elem != 0 && (with_lse || (mask_dtype != -1 && (dtype == CMPEXT3_DTYPE_F32 || elem < 4))))
    return CMPEXT3_E_ALIGN;
  cmpext3::FwdParams p;
  memset(&p, 0, sizeof p);
  const int64_t rs = elem ? D : (D + 7) / 8 * 8;  // element row stride of the dry run's layout
  p.q_s = p.o_s = p.k_s = p.v_s = rs;
  p.q_h = p.o_h = (int64_t)Sq * rs;
  p.k_h = p.v_h = (int64_t)Sk * rs;
  p.q_b = p.o_b = (int64_t)H * Sq * rs;
  p.k_b = p.v_b = (int64_t)H_kv * Sk * rs;
  p.B = B; p.H = H; p.Sq = Sq; p.Sk = Sk; p.D = D;
  p.kv_group = H / H_kv;
  p.mask_kind = mask_dtype == -1 ? cmpext3::MASK_NONE : mask_kind_of(mask_dtype);
  p.lse = with_lse ? (float*)&info : nullptr;  // never dereferenced: marks the training forward
  p.c = 0.125f;
  p.workspace_bytes = workspace_bytes;
  p.elem_rows = elem;
  p.dry = &info;
  hipError_t err;
  if (dtype == CMPEXT3_DTYPE_F32)
    err = cmpext3::launch_mfma32(p, causal != 0, nullptr);
  else
    err = cmpext3::launch_mfma16(p, dtype == CMPEXT3_DTYPE_BF16, causal != 0, nullptr);
  return err == hipSuccess ? CMPEXT3_OK : CMPEXT3_E_INVALID;
}

}  // namespace

extern "C" {

size_t cmpext3_attn_fwd_workspace_size(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                                       int mask_dtype, int causal, int with_lse) {
  // the largest need over every row layout a call may arrive in: whole
  // aligned chunks, and the 4- and 2-byte piece variants (narrow rows)
  size_t need = 0;
  for (int elem : {0, 4, 2}) {
    cmpext3::SplitInfo info;
    if (plan_impl(dtype, B, H, H_kv, Sq, Sk, D, mask_dtype, causal, with_lse, elem, SIZE_MAX, info) ==
            CMPEXT3_OK &&
        info.need > need)
      need = info.need;
  }
  return need;
}

int cmpext3_attn_fwd_plan(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D, int mask_dtype,
                          int causal, int with_lse, size_t workspace_bytes, int* key_parts) {
  cmpext3::SplitInfo info;
  const int es = elem_size(dtype);
  const int elem = es && D * es % 16 != 0 ? (D * es % 4 == 0 ? 4 : 2) : 0;
  const int rc = plan_impl(dtype, B, H, H_kv, Sq, Sk, D, mask_dtype, causal, with_lse, elem,
                           workspace_bytes, info);
  if (key_parts) *key_parts = rc == CMPEXT3_OK ? info.parts : 0;
  return rc;
}

int cmpext3_attn_fwd_ws(const void* q, const void* k, const void* v, void* o, int dtype, int B, int H,
                        int H_kv, int Sq, int Sk, int D, const int64_t q_str[3], const int64_t k_str[3],
                        const int64_t v_str[3], const int64_t o_str[3], const void* mask, int mask_dtype,
                        const int64_t mask_str[3], float scale, int causal, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  return fwd_impl(q, k, v, o, nullptr, dtype, B, H, H_kv, Sq, Sk, D, q_str, k_str, v_str, o_str, mask,
                  mask_dtype, mask_str, scale, causal, stream, workspace, workspace_bytes);
}

int cmpext3_attn_fwd_masked(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                            int H, int H_kv, int Sq, int Sk, int D, const int64_t q_str[3],
                            const int64_t k_str[3], const int64_t v_str[3], const int64_t o_str[3],
                            const void* mask, int mask_dtype, const int64_t mask_str[3], float scale,
                            int causal, hipStream_t stream) {
  return fwd_impl(q, k, v, o, nullptr, dtype, B, H, H_kv, Sq, Sk, D, q_str, k_str, v_str, o_str, mask,
                  mask_dtype, mask_str, scale, causal, stream, nullptr, 0);
}

int cmpext3_attn_fwd_noalloc(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                             int H, int H_kv, int Sq, int Sk, int D, const int64_t q_str[3],
                             const int64_t k_str[3], const int64_t v_str[3], const int64_t o_str[3],
                             const void* mask, int mask_dtype, const int64_t mask_str[3], float scale,
                             int causal, hipStream_t stream) {
  return fwd_impl(q, k, v, o, nullptr, dtype, B, H, H_kv, Sq, Sk, D, q_str, k_str, v_str, o_str, mask,
                  mask_dtype, mask_str, scale, causal, stream, nullptr, 0, /*fixed_exchange=*/true);
}

int cmpext3_attn_fwd_lse(const void* q, const void* k, const void* v, void* o, float* lse, int dtype,
                         int B, int H, int H_kv, int Sq, int Sk, int D, const int64_t q_str[3],
                         const int64_t k_str[3], const int64_t v_str[3], const int64_t o_str[3],
                         const void* mask, int mask_dtype, const int64_t mask_str[3], float scale,
                         int causal, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int rc = check_shape(dtype, B, H, Sq, Sk, D);
  if (rc != CMPEXT3_OK) return rc;
  if ((int64_t)B * H * Sq == 0) return CMPEXT3_OK;
  if (!lse || ((uintptr_t)lse & 3u) != 0) return CMPEXT3_E_INVALID;
  if (!k_str || !v_str) return CMPEXT3_E_INVALID;
  // the pipelined kernel (the one that writes the log-sum-exp up to D = 128)
  // addresses K/V tiles with 32-bit buffer offsets, and the backward that consumes this
  // forward's state does the same for Q and dO (dO takes O's layout): refuse
  // here what cmpext3_attn_bwd would refuse, so no training step can pass the
  // forward and then fail in its backward
  if (!q_str || !o_str) return CMPEXT3_E_INVALID;
  const int es = elem_size(dtype);
  if (!tile_offsets_fit(Sk, k_str[2], v_str[2], es) || !tile_offsets_fit(Sq, q_str[2], o_str[2], es))
    return CMPEXT3_E_TOO_LARGE;
  return fwd_impl(q, k, v, o, lse, dtype, B, H, H_kv, Sq, Sk, D, q_str, k_str, v_str, o_str, mask,
                  mask_dtype, mask_str, scale, causal, stream, workspace, workspace_bytes);
}

size_t cmpext3_attn_bwd_workspace_size(int dtype, int B, int H, int H_kv, int Sq, int Sk, int D,
                                       int mask_dtype, int causal) {
  if (check_shape(dtype, B, H, Sq, Sk, D) != CMPEXT3_OK) return 0;
  if (!whole_chunks(dtype, D) || H_kv < 1 || H_kv > H || H % H_kv != 0) return 0;
  const cmpext3::BwdSplit sp = cmpext3::bwd_split(dtype, B, H, H_kv, Sq, Sk, D, causal != 0, mask_dtype != -1);
  return sp.kv_bytes(B, H_kv, Sk, D) + sp.q_bytes(B, H, Sq, D);
}

int cmpext3_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                     const float* lse, void* dq, void* dk, void* dv, float* delta, int dtype, int B,
                     int H, int H_kv, int Sq, int Sk, int D, const int64_t q_str[3], const int64_t k_str[3],
                     const int64_t v_str[3], const int64_t o_str[3], const int64_t do_str[3],
                     const int64_t dq_str[3], const int64_t dk_str[3], const int64_t dv_str[3],
                     const void* mask, int mask_dtype, const int64_t mask_str[3], float scale, int causal,
                     hipStream_t stream) {
  return cmpext3_attn_bwd_ws(q, k, v, o, dout, lse, dq, dk, dv, delta, dtype, B, H, H_kv, Sq, Sk, D, q_str,
                             k_str, v_str, o_str, do_str, dq_str, dk_str, dv_str, mask, mask_dtype, mask_str,
                             scale, causal, nullptr, 0, stream);
}

int cmpext3_attn_bwd_ws(const void* q, const void* k, const void* v, const void* o, const void* dout,
                        const float* lse, void* dq, void* dk, void* dv, float* delta, int dtype, int B,
                        int H, int H_kv, int Sq, int Sk, int D, const int64_t q_str[3], const int64_t k_str[3],
                        const int64_t v_str[3], const int64_t o_str[3], const int64_t do_str[3],
                        const int64_t dq_str[3], const int64_t dk_str[3], const int64_t dv_str[3],
                        const void* mask, int mask_dtype, const int64_t mask_str[3], float scale, int causal,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
  int rc = check_shape(dtype, B, H, Sq, Sk, D);
  if (rc != CMPEXT3_OK) return rc;
  if ((int64_t)B * H * Sq == 0) return CMPEXT3_OK;
  if (!whole_chunks(dtype, D)) return CMPEXT3_E_HEAD_DIM;
  if (H_kv < 1 || H_kv > H || H % H_kv != 0) return CMPEXT3_E_INVALID;
  bool runs_ok = true;
  rc = check_mask(mask, mask_dtype, mask_str, Sq, Sk, &runs_ok);
  if (rc != CMPEXT3_OK) return rc;
  if (!runs_ok) return CMPEXT3_E_ALIGN;  // the backward reads runs of 8 keys
  if (!q || !k || !v || !o || !dout || !lse || !dq || !dk || !dv || !delta) return CMPEXT3_E_INVALID;
  if (!q_str || !k_str || !v_str || !o_str || !do_str || !dq_str || !dk_str || !dv_str)
    return CMPEXT3_E_INVALID;
  if (!isfinite(scale)) return CMPEXT3_E_INVALID;
  if (((uintptr_t)lse & 3u) != 0 || ((uintptr_t)delta & 3u) != 0) return CMPEXT3_E_ALIGN;
  if (workspace && !aligned16(workspace)) return CMPEXT3_E_ALIGN;
  const void* ptrs[] = {q, k, v, o, dout, dq, dk, dv};
  for (const void* ptr : ptrs)
    if (!aligned16(ptr)) return CMPEXT3_E_ALIGN;
  const int es = elem_size(dtype);
  if (!stride_ok(q_str, B, H, Sq, es) || !stride_ok(o_str, B, H, Sq, es) || !stride_ok(do_str, B, H, Sq, es) ||
      !stride_ok(dq_str, B, H, Sq, es) || !stride_ok(k_str, B, H_kv, Sk, es) || !stride_ok(v_str, B, H_kv, Sk, es) ||
      !stride_ok(dk_str, B, H_kv, Sk, es) || !stride_ok(dv_str, B, H_kv, Sk, es))
    return CMPEXT3_E_ALIGN;
  // Q/dO tiles (dK/dV kernel) and K/V tiles (dQ kernel) use 32-bit buffer offsets
  if (!tile_offsets_fit(Sq, q_str[2], do_str[2], es) || !tile_offsets_fit(Sk, k_str[2], v_str[2], es))
    return CMPEXT3_E_TOO_LARGE;

  cmpext3::BwdParams p;
  memset(&p, 0, sizeof p);
  p.q = q; p.k = k; p.v = v; p.o = o; p.dout = dout; p.lse = lse;
  p.dq = dq; p.dk = dk; p.dv = dv; p.delta = delta;
  p.q_b = q_str[0]; p.q_h = q_str[1]; p.q_s = q_str[2];
  p.k_b = k_str[0]; p.k_h = k_str[1]; p.k_s = k_str[2];
  p.v_b = v_str[0]; p.v_h = v_str[1]; p.v_s = v_str[2];
  p.o_b = o_str[0]; p.o_h = o_str[1]; p.o_s = o_str[2];
  p.do_b = do_str[0]; p.do_h = do_str[1]; p.do_s = do_str[2];
  p.dq_b = dq_str[0]; p.dq_h = dq_str[1]; p.dq_s = dq_str[2];
  p.dk_b = dk_str[0]; p.dk_h = dk_str[1]; p.dk_s = dk_str[2];
  p.dv_b = dv_str[0]; p.dv_h = dv_str[1]; p.dv_s = dv_str[2];
  p.B = B; p.H = H; p.Sq = Sq; p.Sk = Sk; p.D = D;
  p.Hkv = H_kv;
  p.group = H / H_kv;
  p.mask_kind = cmpext3::MASK_NONE;
  if (mask_dtype != -1) {
    p.mask = mask;
    p.m_b = mask_str[0]; p.m_h = mask_str[1]; p.m_q = mask_str[2];
    p.mask_kind = mask_kind_of(mask_dtype);
  }
  // The fp16/bf16 dK/dV kernel divides by c.  For |scale| * log2(e) below 1e-30 (scale 0
  // and denormal scales) c = 1e-30 moves each exp2 argument by at most
  // 1e-30 * |score|, and keeps -lse2 / c finite
  p.c = fmaxf(fabsf(scale) * cmpext3::kLog2e, 1e-30f);
  p.scale = scale;
  p.sign = scale < 0.f ? (dtype == CMPEXT3_DTYPE_F32 ? 0x80000000u : 0x80008000u) : 0u;
  // split sweeps where the workspace holds their partials (dK/dV first, then
  // dQ; a sweep whose partials do not fit runs unsplit)
  p.nsplit = p.nsplit_q = 1;
  if (workspace) {
    const cmpext3::BwdSplit sp =
        cmpext3::bwd_split(dtype, B, H, H_kv, Sq, Sk, D, causal != 0, p.mask_kind != cmpext3::MASK_NONE);
    const size_t kvb = sp.kv_bytes(B, H_kv, Sk, D), qb = sp.q_bytes(B, H, Sq, D);
    size_t used = 0;
    if (kvb > 0 && kvb <= workspace_bytes) {
      p.nsplit = sp.ns_kv;
      p.nfull = sp.nfull_kv;
      p.part = (float*)workspace;
      used = kvb;
    }
    if (qb > 0 && used + qb <= workspace_bytes) {
      p.nsplit_q = sp.ns_q;
      p.nfull_q = sp.nfull_q;
      p.part_q = (float*)((char*)workspace + used);
    }
  }
  const hipError_t err = dtype == CMPEXT3_DTYPE_F32
                             ? cmpext3::launch_bwd32(p, causal != 0, stream)
                             : cmpext3::launch_bwd16(p, dtype == CMPEXT3_DTYPE_BF16, causal != 0, stream);
  return err == hipSuccess ? CMPEXT3_OK : CMPEXT3_E_LAUNCH;
}

}  // extern "C"
