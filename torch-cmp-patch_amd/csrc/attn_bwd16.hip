// Launch sequence of the attention backward (templates in attn_bwd16.h):
// Delta, then dK/dV over key blocks, then dQ over query blocks, all on the
// caller's stream.  Head dims up to 64 use the 64 bucket, up to 128 the 128
// bucket, up to 192 and 256 those (columns past D are zero in every operand
// and never stored).
#include "attn_bwd16.h"

namespace cmpext3 {

namespace {

template <typename T, int DK, bool CAUSAL, bool MASK>
hipError_t launch_bwd_t(const BwdParams& p0, hipStream_t s) {
  BwdParams p = p0;
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  hipLaunchKernelGGL(attn_bwd_delta<T>, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, p);
  p.n_blk = (p.Sk + 127) / 128;
  p.n_wg = p.B * p.Hkv * p.n_blk;
  hipLaunchKernelGGL((attn_bwd_dkdv<T, DK, CAUSAL, MASK>), dim3(p.n_wg), dim3(256), 0, s, p);
  p.n_blk = (p.Sq + 127) / 128;
  p.n_wg = p.B * p.H * p.n_blk;
  hipLaunchKernelGGL((attn_bwd_dq<T, DK, CAUSAL, MASK>), dim3(p.n_wg), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, bool MASK>
hipError_t launch_bwd_mask(const BwdParams& p, int dk, bool causal, hipStream_t s) {
  if (dk == 64) return causal ? launch_bwd_t<T, 64, true, MASK>(p, s) : launch_bwd_t<T, 64, false, MASK>(p, s);
  if (dk == 128) return causal ? launch_bwd_t<T, 128, true, MASK>(p, s) : launch_bwd_t<T, 128, false, MASK>(p, s);
  if (dk == 192) return causal ? launch_bwd_t<T, 192, true, MASK>(p, s) : launch_bwd_t<T, 192, false, MASK>(p, s);
  if (dk == 256) return causal ? launch_bwd_t<T, 256, true, MASK>(p, s) : launch_bwd_t<T, 256, false, MASK>(p, s);
  return hipErrorNotSupported;
}

template <typename T>
hipError_t launch_bwd_dtype(const BwdParams& p, int dk, bool causal, hipStream_t s) {
  return p.mask_kind != MASK_NONE ? launch_bwd_mask<T, true>(p, dk, causal, s)
                                  : launch_bwd_mask<T, false>(p, dk, causal, s);
}

}  // namespace

int bwd16_bucket(int D) { return D <= 0 ? -1 : D <= 64 ? 64 : D <= 128 ? 128 : D <= 192 ? 192 : D <= 256 ? 256 : -1; }

hipError_t launch_bwd16(const BwdParams& p, bool bf16, bool causal, hipStream_t s) {
  if ((int64_t)p.B * p.H * p.Sq == 0) return hipSuccess;
  const int dk = bwd16_bucket(p.D);
  return bf16 ? launch_bwd_dtype<__bf16>(p, dk, causal, s) : launch_bwd_dtype<_Float16>(p, dk, causal, s);
}

}  // namespace cmpext3
