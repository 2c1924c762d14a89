// Instantiations of the software-pipelined fp16/bf16 kernel (template in
// attn_fwd_pipe16.h) for head dims above 128 with an attention mask (OPT bit
// 16; buckets 160, 192, 256) or the row log-sum-exp of the training forward
// (OPT bit 32; buckets 192 and 256, masked or not): one wave per SIMD, K/V
// straight into LDS with padded rows, Q never pre-scaled (one instantiation
// per dtype serves every scale).  Plan and dispatch in attn_fwd_pipe16.hip.
#include "attn_fwd_pipe16.h"

namespace cmpext3 {

namespace {

template <typename T, int DK, bool CAUSAL, int MOPT>
hipError_t launch_wm_dk(const FwdParams& p, const SplitArgs& sa, hipStream_t s) {
  return launch_pipe16_cfg<T, DK, 4, 32, 1, CAUSAL, false, 1 | 8 | 256 | MOPT>(p, sa, s);
}

template <typename T, bool CAUSAL>
hipError_t launch_wm(const FwdParams& p, const SplitArgs& sa, int dk, hipStream_t s) {
  const bool m = p.mask_kind != MASK_NONE;
  if (p.lse) {
    if (dk == 192) return m ? launch_wm_dk<T, 192, CAUSAL, 48>(p, sa, s) : launch_wm_dk<T, 192, CAUSAL, 32>(p, sa, s);
    if (dk == 256) return m ? launch_wm_dk<T, 256, CAUSAL, 48>(p, sa, s) : launch_wm_dk<T, 256, CAUSAL, 32>(p, sa, s);
    return hipErrorNotSupported;
  }
  switch (dk) {
    case 160: return launch_wm_dk<T, 160, CAUSAL, 16>(p, sa, s);
    case 192: return launch_wm_dk<T, 192, CAUSAL, 16>(p, sa, s);
    case 256: return launch_wm_dk<T, 256, CAUSAL, 16>(p, sa, s);
  }
  return hipErrorNotSupported;
}

}  // namespace

hipError_t launch_pipe16_wide_mt(const FwdParams& p, const SplitArgs& sa, int dk, bool bf16, bool causal,
                                 hipStream_t s) {
  if (bf16) return causal ? launch_wm<__bf16, true>(p, sa, dk, s) : launch_wm<__bf16, false>(p, sa, dk, s);
  return causal ? launch_wm<_Float16, true>(p, sa, dk, s) : launch_wm<_Float16, false>(p, sa, dk, s);
}

}  // namespace cmpext3
