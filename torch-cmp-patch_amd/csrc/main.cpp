// cmpext3._native -- torch binding of the fused attention forward.
//
// attention(query, key, value, scale=None, causal=False, attn_mask=None) -> Tensor
//   Same signature and error convention as the reference's binding
//   (src/main.cpp:2353-2358 -> custom_attention_forward, :1603-1774): every
//   unsupported input raises RuntimeError (TORCH_CHECK) so that the Python
//   patch falls back to stock SDPA.  The compute goes through the C ABI in
//   include/cmpext3_attn.h on the caller's current stream.
//
// Differences from the reference binding, by design:
//   * bf16 runs natively (the reference casts bf16 -> fp16 -> bf16, :1623-1627);
//   * causal, Sq != Sk and strided inputs are accepted for every dtype;
//   * a [B,S,H,D]-memory query (diffusers/webui layout viewed as [B,H,S,D])
//     gets its output in [B,S,H,D] memory too, returned as the same kind of
//     view (the reference's HFMA2 path does this for fp16, :1652);
//   * head dims that are not a whole number of 16-byte chunks, and tensors
//     whose base pointer or row strides are not 16-byte aligned, run in place
//     (narrow-row kernel variants); 16-bit rows with an odd element count or
//     offset (2-byte pieces, slower in place than copied), and masked fp32
//     rows off whole 16-byte chunks, repack such inputs into zero-padded
//     contiguous copies;
//   * K/V may hold fewer heads than Q (grouped-query attention);
//   * attn_mask (bool or additive f16/bf16/f32, broadcast like torch's SDPA)
//     runs natively for every dtype and head dim, alone or combined with
//     causal (the reference sent every mask to stock torch,
//     cmpext3/__init__.py:624).
//
// attention_fwd_lse / attention_bwd: the training pair (no reference
// counterpart: the reference is forward-only, cmpext3/__init__.py:115-125),
// used by cmpext3's autograd Function.
#include <cmath>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include <torch/extension.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include "../../include/cmpext3_attn.h"

namespace {

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kHalf: return CMPEXT3_DTYPE_F16;
    case at::kBFloat16: return CMPEXT3_DTYPE_BF16;
    case at::kFloat: return CMPEXT3_DTYPE_F32;
    default: return -1;
  }
}

// attention mask in the form the C ABI takes: [B,H,Sq,Sk] view, unit key
// stride, other strides multiples of 4 elements (0 = broadcast)
struct Mask {
  torch::Tensor t;
  int dtype = -1;
};

// Key-split workspace of one (device, stream): a byte tensor from torch's
// caching allocator (so torch.cuda.memory_allocated counts it), zero-filled
// when made -- its first 64 KiB are the counters every launch leaves at zero
// -- and kept for later calls on the stream, replaced by a larger one when a
// bigger plan arrives.  Calls on one stream run in order, so they can share
// it.  A stream under graph capture gets none and its launch runs unsplit: a
// captured launch would carry the buffer into replays that can run beside
// eager calls on the stream.
struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};

std::mutex ws_mu;
std::map<std::pair<int, hipStream_t>, torch::Tensor> ws_cache;  // guarded by ws_mu

Workspace workspace_for(const torch::Tensor& like, hipStream_t stream, size_t need) {
  Workspace w;
  if (need == 0) return w;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess) {
    (void)hipGetLastError();
    return w;
  }
  if (cap != hipStreamCaptureStatusNone) return w;
  std::lock_guard<std::mutex> lock(ws_mu);
  torch::Tensor& t = ws_cache[std::make_pair((int)like.get_device(), stream)];
  if (!t.defined() || (size_t)t.numel() < need)
    t = torch::zeros({(int64_t)need}, like.options().dtype(at::kByte));
  w.ptr = t.data_ptr();
  w.bytes = (size_t)t.numel();
  return w;
}

size_t workspace_size_of(int device, hipStream_t stream) {
  std::lock_guard<std::mutex> lock(ws_mu);
  const auto it = ws_cache.find(std::make_pair(device, stream));
  return it == ws_cache.end() ? 0 : (size_t)it->second.numel();
}

int launch(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
           torch::Tensor& o, int dtype, int D, float scale, bool causal, const Mask& mask,
           hipStream_t stream) {
  const int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
  const int64_t ks[3] = {k.stride(0), k.stride(1), k.stride(2)};
  const int64_t vs[3] = {v.stride(0), v.stride(1), v.stride(2)};
  const int64_t os[3] = {o.stride(0), o.stride(1), o.stride(2)};
  if (q.stride(3) != 1 || k.stride(3) != 1 || v.stride(3) != 1 || o.stride(3) != 1)
    return CMPEXT3_E_ALIGN;
  int64_t ms[3] = {0, 0, 0};
  if (mask.dtype >= 0) {
    ms[0] = mask.t.stride(0); ms[1] = mask.t.stride(1); ms[2] = mask.t.stride(2);
  }
  const int B = (int)q.size(0), H = (int)q.size(1), Hkv = (int)k.size(1), Sq = (int)q.size(2),
            Sk = (int)k.size(2);
  const Workspace ws = workspace_for(
      q, stream, cmpext3_attn_fwd_workspace_size(dtype, B, H, Hkv, Sq, Sk, D, mask.dtype, causal ? 1 : 0, 0));
  return cmpext3_attn_fwd_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), dtype, B, H, Hkv, Sq,
                             Sk, D, qs, ks, vs, os, mask.dtype >= 0 ? mask.t.data_ptr() : nullptr,
                             mask.dtype, ms, scale, causal ? 1 : 0, ws.ptr, ws.bytes, stream);
}

// torch's attn_mask broadcast to [B,H,Sq,Sk]; copied into a compact buffer
// (broadcast dims kept at size 1, rows padded to a multiple of 8 keys) when
// its layout does not fit the ABI.  Inference calls (runs == false) need
// only a unit key stride: the ABI reads any other layout element by element.
// Training calls (runs == true) need rows readable in runs of 8 keys.
Mask prepare_mask(const torch::Tensor& m0, const torch::Tensor& query, int64_t B, int64_t H,
                  int64_t Sq, int64_t Sk, bool runs) {
  TORCH_CHECK(m0.device() == query.device(), "cmpext3 attention: attn_mask on another device");
  TORCH_CHECK(m0.dim() <= 4, "cmpext3 attention: attn_mask has more than 4 dims");
  Mask mk;
  switch (m0.scalar_type()) {
    case at::kBool: mk.dtype = CMPEXT3_DTYPE_BOOL; break;
    case at::kHalf: mk.dtype = CMPEXT3_DTYPE_F16; break;
    case at::kBFloat16: mk.dtype = CMPEXT3_DTYPE_BF16; break;
    case at::kFloat: mk.dtype = CMPEXT3_DTYPE_F32; break;
    default: TORCH_CHECK(false, "cmpext3 attention: unsupported attn_mask dtype ", m0.scalar_type());
  }
  torch::Tensor m = m0.expand({B, H, Sq, Sk});
  // in place only if rows can be read in runs of 8 keys without leaving the
  // tensor: unit key stride and Sk a multiple of 8
  const bool fits = m.stride(3) == 1 &&
                    (!runs || (Sk % 8 == 0 && m.stride(0) % 4 == 0 && m.stride(1) % 4 == 0 &&
                               m.stride(2) % 4 == 0 && ((uintptr_t)m.data_ptr() & 15u) == 0));
  if (!fits) {
    const int64_t cb = m.stride(0) == 0 ? 1 : B, ch = m.stride(1) == 0 ? 1 : H;
    const int64_t cq = m.stride(2) == 0 ? 1 : Sq, skp = (Sk + 7) / 8 * 8;
    torch::Tensor c = torch::zeros({cb, ch, cq, skp}, m.options());
    c.narrow(3, 0, Sk).copy_(m.narrow(0, 0, cb).narrow(1, 0, ch).narrow(2, 0, cq));
    m = c.narrow(3, 0, Sk).expand({B, H, Sq, Sk});
  }
  mk.t = m;
  return mk;
}

// Would the C ABI read these rows in 2-byte pieces?  True for 16-bit dtypes
// when the row length, a base pointer or a row stride is an odd number of
// 16-bit elements (the ABI's piece size is the largest of 2/4/8/16 bytes
// dividing all of them).
bool two_byte_rows(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                   const torch::Tensor& o, int64_t D) {
  if (q.element_size() != 2) return false;
  uint64_t bits = (uint64_t)D * 2;
  for (const torch::Tensor* t : {&q, &k, &v, &o}) {
    bits |= (uintptr_t)t->data_ptr();
    for (int i = 0; i < 3; ++i)
      if (t->size(i) > 1) bits |= (uint64_t)t->stride(i) * 2;
  }
  return (bits & 3) != 0;
}

bool is_bshd_view(const torch::Tensor& t) {
  // [B,H,S,D] view of [B,S,H,D] memory
  const int64_t H = t.size(1), S = t.size(2), D = t.size(3);
  return H > 1 && S > 1 && t.stride(3) == 1 && t.stride(1) == D && t.stride(2) == H * D &&
         t.stride(0) == S * H * D;
}

}  // namespace

torch::Tensor attention(torch::Tensor query, torch::Tensor key, torch::Tensor value,
                        c10::optional<double> scale_arg, bool causal,
                        c10::optional<torch::Tensor> attn_mask) {
  TORCH_CHECK(query.dim() == 4, "cmpext3 attention: query must be 4D [B, H, S, D]");
  TORCH_CHECK(key.dim() == 4, "cmpext3 attention: key must be 4D");
  TORCH_CHECK(value.dim() == 4, "cmpext3 attention: value must be 4D");
  TORCH_CHECK(query.is_cuda() && key.is_cuda() && value.is_cuda(),
              "cmpext3 attention: tensors must be on the GPU");
  TORCH_CHECK(query.device() == key.device() && query.device() == value.device(),
              "cmpext3 attention: device mismatch");
  TORCH_CHECK(query.scalar_type() == key.scalar_type() && query.scalar_type() == value.scalar_type(),
              "cmpext3 attention: q, k, v must share one dtype");
  const int dtype = dtype_code(query.scalar_type());
  TORCH_CHECK(dtype >= 0, "cmpext3 attention: unsupported dtype ", query.scalar_type());

  const int64_t B = query.size(0), H = query.size(1), Sq = query.size(2), D = query.size(3);
  const int64_t Sk = key.size(2), Hkv = key.size(1);
  // K/V may hold fewer heads than Q when that count divides H (grouped-query
  // attention, torch's enable_gqa semantics: query head h uses K/V head
  // h / (H / Hkv)); the Python patch only sends such calls with enable_gqa.
  TORCH_CHECK(key.size(0) == B && key.size(3) == D && (Hkv == H || (Hkv >= 1 && H % Hkv == 0)),
              "cmpext3 attention: key shape mismatch");
  TORCH_CHECK(value.size(0) == B && value.size(1) == Hkv && value.size(2) == Sk && value.size(3) == D,
              "cmpext3 attention: value shape mismatch");
  TORCH_CHECK(D >= 1 && D <= 256, "cmpext3 attention: head dim ", D, " outside 1..256");
  TORCH_CHECK(Sk > 0 || B * H * Sq == 0, "cmpext3 attention: empty key sequence");

  const float scale = scale_arg.has_value() ? (float)scale_arg.value()
                                            : 1.0f / std::sqrt((float)D);
  TORCH_CHECK(std::isfinite(scale), "cmpext3 attention: non-finite scale");

  const at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.device().index()).stream();

  Mask mask;
  if (attn_mask.has_value() && attn_mask->defined()) {
    mask = prepare_mask(*attn_mask, query, B, H, Sq, Sk, false);
  }

  torch::Tensor out = is_bshd_view(query)
                          ? torch::empty({B, Sq, H, D}, query.options()).transpose(1, 2)
                          : torch::empty({B, H, Sq, D}, query.options());
  if (out.numel() == 0) return out;

  // Rows the C ABI would read in 2-byte pieces (f16/bf16 with an odd head dim
  // or an odd element offset) go through the padded copy below instead: on
  // MI355X the copies plus the vector-load kernel take about a third of the
  // time of the in-place 2-byte path (D = 33: 45 us against 123 us).
  int rc = two_byte_rows(query, key, value, out, D)
               ? CMPEXT3_E_ALIGN
               : launch(query, key, value, out, dtype, (int)D, scale, causal, mask, stream);
  if (rc == CMPEXT3_E_ALIGN || rc == CMPEXT3_E_HEAD_DIM) {
    // 2-byte rows, and masked rows the ABI refuses (fp32 off whole chunks;
    // it runs any other layout in place): repack into contiguous copies
    // zero-padded to whole 16-byte chunks.
    // Zero columns add nothing to Q K^T, and the padded V columns only produce
    // output columns that are cut away again; `scale` already used the true D.
    const int64_t chunk = (dtype == CMPEXT3_DTYPE_F32) ? 4 : 8;
    const int64_t Dp = (D + chunk - 1) / chunk * chunk;
    TORCH_CHECK(Dp <= 256, "cmpext3 attention: padded head dim ", Dp, " exceeds 256");
    auto pad = [&](const torch::Tensor& t) {
      return Dp == D ? t.clone(at::MemoryFormat::Contiguous)
                     : at::constant_pad_nd(t, {0, Dp - D}, 0).contiguous();
    };
    torch::Tensor qp = pad(query), kp = pad(key), vp = pad(value);
    torch::Tensor op = torch::empty({B, H, Sq, Dp}, query.options());
    rc = launch(qp, kp, vp, op, dtype, (int)Dp, scale, causal, mask, stream);
    if (rc == CMPEXT3_OK) out = (Dp == D) ? op : op.narrow(3, 0, D).contiguous();
  }
  TORCH_CHECK(rc == CMPEXT3_OK, "cmpext3 attention: ", cmpext3_attn_strerror(rc));
  return out;
}

namespace {

// Shared checks of the training entry points: 4-D GPU f16/bf16/fp32 tensors of
// one dtype and device, K/V heads dividing the query heads, head dim <= 256.
int training_dtype(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v) {
  TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "cmpext3 attention: q, k, v must be 4D");
  TORCH_CHECK(q.is_cuda() && q.device() == k.device() && q.device() == v.device(),
              "cmpext3 attention: tensors must be on one GPU");
  TORCH_CHECK(q.scalar_type() == k.scalar_type() && q.scalar_type() == v.scalar_type(),
              "cmpext3 attention: q, k, v must share one dtype");
  const int dtype = dtype_code(q.scalar_type());
  TORCH_CHECK(dtype == CMPEXT3_DTYPE_F16 || dtype == CMPEXT3_DTYPE_BF16 || dtype == CMPEXT3_DTYPE_F32,
              "cmpext3 attention: the training path takes fp16/bf16/fp32 only");
  TORCH_CHECK(k.size(0) == q.size(0) && k.size(1) >= 1 && q.size(1) % k.size(1) == 0 &&
                  k.size(3) == q.size(3) && v.sizes() == k.sizes(),
              "cmpext3 attention: the training path needs K/V of Q's batch and head dim, with a "
              "head count dividing Q's");
  TORCH_CHECK(q.size(3) >= 1 && q.size(3) <= 256, "cmpext3 attention: the training path needs D <= 256");
  TORCH_CHECK(k.size(2) > 0 || q.size(0) * q.size(1) * q.size(2) == 0,
              "cmpext3 attention: empty key sequence");
  return dtype;
}

// The ABI's training layout: unit head-dim stride, 16-byte aligned base and
// row strides, head dim a whole number of 16-byte chunks (zero-padded to Dp
// otherwise).
torch::Tensor abi_layout(const torch::Tensor& t, int64_t Dp) {
  const int64_t D = t.size(3);
  if (Dp != D) return at::constant_pad_nd(t, {0, Dp - D}, 0).contiguous();
  const int64_t chunk = 16 / t.element_size();
  const bool ok = t.stride(3) == 1 && ((uintptr_t)t.data_ptr() & 15u) == 0 && t.stride(0) % chunk == 0 &&
                  t.stride(1) % chunk == 0 && t.stride(2) % chunk == 0;
  return ok ? t : t.contiguous();
}

// Head dim padded to whole 16-byte chunks of the training dtype.
int64_t chunk_dim(const torch::Tensor& t) {
  const int64_t chunk = 16 / t.element_size();
  return (t.size(3) + chunk - 1) / chunk * chunk;
}

void strides3(const torch::Tensor& t, int64_t s[3]) {
  s[0] = t.stride(0); s[1] = t.stride(1); s[2] = t.stride(2);
}

float resolve_scale(c10::optional<double> scale_arg, int64_t D) {
  const float scale = scale_arg.has_value() ? (float)scale_arg.value() : 1.0f / std::sqrt((float)D);
  TORCH_CHECK(std::isfinite(scale), "cmpext3 attention: non-finite scale");
  return scale;
}

}  // namespace

// Training forward: (out, lse), lse = [B, H, Sq] fp32 natural-log row
// log-sum-exp, the state attention_bwd needs.
std::vector<torch::Tensor> attention_fwd_lse(torch::Tensor query, torch::Tensor key, torch::Tensor value,
                                             c10::optional<double> scale_arg, bool causal,
                                             c10::optional<torch::Tensor> attn_mask) {
  const int dtype = training_dtype(query, key, value);
  const int64_t B = query.size(0), H = query.size(1), Sq = query.size(2), D = query.size(3);
  const int64_t Sk = key.size(2), Hkv = key.size(1), Dp = chunk_dim(query);
  const float scale = resolve_scale(scale_arg, D);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.device().index()).stream();

  torch::Tensor lse = torch::empty({B, H, Sq}, query.options().dtype(at::kFloat));
  torch::Tensor out = torch::empty({B, H, Sq, Dp}, query.options());
  if (out.numel() == 0) return {Dp == D ? out : out.narrow(3, 0, D), lse};
  Mask mask;
  int64_t ms[3] = {0, 0, 0};
  if (attn_mask.has_value() && attn_mask->defined()) {
    mask = prepare_mask(*attn_mask, query, B, H, Sq, Sk, true);
    strides3(mask.t, ms);
  }
  const torch::Tensor q = abi_layout(query, Dp), k = abi_layout(key, Dp), v = abi_layout(value, Dp);
  int64_t qs[3], ks[3], vs[3], os[3];
  strides3(q, qs); strides3(k, ks); strides3(v, vs); strides3(out, os);
  const Workspace ws = workspace_for(
      query, stream,
      cmpext3_attn_fwd_workspace_size(dtype, (int)B, (int)H, (int)Hkv, (int)Sq, (int)Sk, (int)Dp, mask.dtype,
                                      causal ? 1 : 0, 1));
  const int rc = cmpext3_attn_fwd_lse(q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                                      lse.data_ptr<float>(), dtype, (int)B, (int)H, (int)Hkv, (int)Sq,
                                      (int)Sk, (int)Dp, qs, ks, vs, os,
                                      mask.dtype >= 0 ? mask.t.data_ptr() : nullptr, mask.dtype, ms, scale,
                                      causal ? 1 : 0, ws.ptr, ws.bytes, stream);
  TORCH_CHECK(rc == CMPEXT3_OK, "cmpext3 attention: ", cmpext3_attn_strerror(rc));
  return {Dp == D ? out : out.narrow(3, 0, D).contiguous(), lse};
}

// Training backward: (dq, dk, dv) of sum(out * grad_out) for out =
// attention_fwd_lse(query, key, value, scale, causal)[0].
std::vector<torch::Tensor> attention_bwd(torch::Tensor query, torch::Tensor key, torch::Tensor value,
                                         torch::Tensor out, torch::Tensor grad_out, torch::Tensor lse,
                                         c10::optional<double> scale_arg, bool causal,
                                         c10::optional<torch::Tensor> attn_mask) {
  const int dtype = training_dtype(query, key, value);
  const int64_t B = query.size(0), H = query.size(1), Sq = query.size(2), D = query.size(3);
  const int64_t Sk = key.size(2), Hkv = key.size(1), Dp = chunk_dim(query);
  TORCH_CHECK(out.sizes() == query.sizes() && grad_out.sizes() == query.sizes() &&
                  out.scalar_type() == query.scalar_type() && grad_out.scalar_type() == query.scalar_type(),
              "cmpext3 attention: out / grad_out must match query");
  TORCH_CHECK(lse.scalar_type() == at::kFloat && lse.dim() == 3 && lse.size(0) == B && lse.size(1) == H &&
                  lse.size(2) == Sq,
              "cmpext3 attention: lse must be fp32 [B, H, Sq]");
  TORCH_CHECK(out.device() == query.device() && grad_out.device() == query.device() &&
                  lse.device() == query.device(),
              "cmpext3 attention: tensors must be on one GPU");
  const float scale = resolve_scale(scale_arg, D);
  const at::hip::HIPGuardMasqueradingAsCUDA guard(query.device());
  hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(query.device().index()).stream();

  torch::Tensor dq = torch::empty({B, H, Sq, Dp}, query.options());
  torch::Tensor dk = torch::empty({B, Hkv, Sk, Dp}, query.options());
  torch::Tensor dv = torch::empty({B, Hkv, Sk, Dp}, query.options());
  if (B * H * Sq == 0) {  // no query: nothing reaches K or V
    dk.zero_();
    dv.zero_();
  } else {
    const torch::Tensor q = abi_layout(query, Dp), k = abi_layout(key, Dp), v = abi_layout(value, Dp);
    // dO gets O's row stride limits (32-bit tile offsets); a gradient in an
    // exotic layout is packed rather than refused
    const torch::Tensor o = abi_layout(out, Dp);
    torch::Tensor g = abi_layout(grad_out, Dp);
    if ((Sq + 64) * std::max<int64_t>(g.stride(2), 1) * g.element_size() >= INT32_MAX) g = g.contiguous();
    const torch::Tensor l = lse.contiguous();
    torch::Tensor delta = torch::empty({B, H, Sq}, query.options().dtype(at::kFloat));
    Mask mask;
    int64_t ms[3] = {0, 0, 0};
    if (attn_mask.has_value() && attn_mask->defined()) {
      mask = prepare_mask(*attn_mask, query, B, H, Sq, Sk, true);
      strides3(mask.t, ms);
    }
    int64_t qs[3], ks[3], vs[3], os[3], gs[3], dqs[3], dks[3], dvs[3];
    strides3(q, qs); strides3(k, ks); strides3(v, vs); strides3(o, os); strides3(g, gs);
    strides3(dq, dqs); strides3(dk, dks); strides3(dv, dvs);
    // split dK/dV sweeps (few key blocks for the CUs) sum fp32 partials kept
    // in a workspace from torch's caching allocator, on this stream
    const size_t wsb = cmpext3_attn_bwd_workspace_size(dtype, (int)B, (int)H, (int)Hkv, (int)Sq, (int)Sk,
                                                       (int)Dp, mask.dtype, causal ? 1 : 0);
    torch::Tensor ws;
    if (wsb > 0) ws = torch::empty({(int64_t)wsb}, query.options().dtype(at::kByte));
    const int rc = cmpext3_attn_bwd_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), g.data_ptr(),
                                       l.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                                       delta.data_ptr<float>(), dtype, (int)B, (int)H, (int)Hkv, (int)Sq,
                                       (int)Sk, (int)Dp, qs, ks, vs, os, gs, dqs, dks, dvs,
                                       mask.dtype >= 0 ? mask.t.data_ptr() : nullptr, mask.dtype, ms, scale,
                                       causal ? 1 : 0, wsb > 0 ? ws.data_ptr() : nullptr, wsb, stream);
    TORCH_CHECK(rc == CMPEXT3_OK, "cmpext3 attention backward: ", cmpext3_attn_strerror(rc));
  }
  if (Dp != D) {
    dq = dq.narrow(3, 0, D).contiguous();
    dk = dk.narrow(3, 0, D).contiguous();
    dv = dv.narrow(3, 0, D).contiguous();
  }
  return {dq, dk, dv};
}

int64_t workspace_bytes(int64_t device) {
  const hipStream_t stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA((c10::DeviceIndex)device).stream();
  return (int64_t)workspace_size_of((int)device, stream);
}

std::string describe(int64_t dtype, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                     bool causal) {
  char buf[384];
  cmpext3_attn_describe((int)dtype, (int)B, (int)H, (int)Sq, (int)Sk, (int)D, causal ? 1 : 0, buf,
                        sizeof buf);
  return std::string(buf);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "cmpext3 native ops for MI355X (gfx950): fused attention forward";
  m.def("attention", &attention, "Fused SDPA forward (fp16/bf16/fp32, causal or not)",
        py::arg("query"), py::arg("key"), py::arg("value"), py::arg("scale") = py::none(),
        py::arg("causal") = false, py::arg("attn_mask") = py::none());
  m.def("describe", &describe, "Kernel/tile choice for a problem (host only)", py::arg("dtype"),
        py::arg("B"), py::arg("H"), py::arg("Sq"), py::arg("Sk"), py::arg("D"),
        py::arg("causal") = false);
  m.def("attention_fwd_lse", &attention_fwd_lse,
        "Training forward (fp16/bf16/fp32, D <= 256): returns (out, lse), lse = fp32 [B,H,Sq] row "
        "log-sum-exp (natural log)",
        py::arg("query"), py::arg("key"), py::arg("value"), py::arg("scale") = py::none(),
        py::arg("causal") = false, py::arg("attn_mask") = py::none());
  m.def("attention_bwd", &attention_bwd,
        "Training backward: (dq, dk, dv) from q, k, v, out, grad_out and the forward's lse",
        py::arg("query"), py::arg("key"), py::arg("value"), py::arg("out"), py::arg("grad_out"),
        py::arg("lse"), py::arg("scale") = py::none(), py::arg("causal") = false,
        py::arg("attn_mask") = py::none());
  m.def("abi_version", &cmpext3_attn_abi_version, "C ABI version of libcmpext3_attn.so");
  m.def("workspace_bytes", &workspace_bytes,
        "Bytes of key-split workspace the binding keeps for the current stream of `device` (0: none yet)",
        py::arg("device") = 0);
}
