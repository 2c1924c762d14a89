// Launch sequence of the attention backward (templates in attn_bwd16.h):
// Delta, then dK/dV over key blocks (split sweeps: then the sum of their
// partials), then dQ over query blocks, all on the caller's stream.  Head
// dims up to 64 use the 64 bucket, up to 128 the 128 bucket, up to 192 and
// 256 those (columns past D are zero in every operand and never stored).
#include "attn_bwd16.h"

namespace cmpext3 {

namespace {

template <typename T, int DK, bool CAUSAL, bool MASK>
hipError_t launch_bwd_t(const BwdParams& p0, hipStream_t s) {
  BwdParams p = p0;
  const int64_t rows = (int64_t)p.B * p.H * p.Sq;
  hipLaunchKernelGGL(attn_bwd_delta<T>, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, p);
  p.n_blk = (p.Sk + 127) / 128;
  const int ns = p.nsplit > 1 && p.part ? p.nsplit : 1;
  p.nsplit = ns;
  if (ns == 1 || CAUSAL) p.nfull = 0;
  const int n_kv = p.B * p.Hkv * p.n_blk;
  p.n_wg = p.nfull > 0 ? p.nfull + (n_kv - p.nfull) * ns : n_kv * ns;
  hipLaunchKernelGGL((attn_bwd_dkdv<T, DK, CAUSAL, MASK>), dim3(p.n_wg), dim3(256), 0, s, p);
  if (ns > 1) {
    if (p.nfull > 0) {
      const int64_t n4 = (int64_t)(n_kv - p.nfull) * 128 * p.D / 4;
      hipLaunchKernelGGL((attn_bwd_tail_sum<T, true>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, p);
    } else {
      launch_part_sums<T>(p, true, s);
    }
  }
  p.n_blk = (p.Sq + 127) / 128;
  const int nsq = p.nsplit_q > 1 && p.part_q ? p.nsplit_q : 1;
  p.nsplit_q = nsq;
  if (nsq == 1 || CAUSAL) p.nfull_q = 0;
  const int n_q = p.B * p.H * p.n_blk;
  p.n_wg = p.nfull_q > 0 ? p.nfull_q + (n_q - p.nfull_q) * nsq : n_q * nsq;
  hipLaunchKernelGGL((attn_bwd_dq<T, DK, CAUSAL, MASK>), dim3(p.n_wg), dim3(256), 0, s, p);
  if (nsq > 1) {
    if (p.nfull_q > 0) {
      const int64_t n4 = (int64_t)(n_q - p.nfull_q) * 128 * p.D / 4;
      hipLaunchKernelGGL((attn_bwd_tail_sum<T, false>), dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, p);
    } else {
      launch_part_sums<T>(p, false, s);
    }
  }
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

// Split plan of the f16/bf16 gradient sweeps (split_sweep): dK/dV over
// 128-key blocks, each sweeping (query head of the group, 32-query tile);
// dQ over 128-query blocks, each sweeping 32-key tiles.  Workgroups per CU
// follow the kernels' waves per SIMD.
BwdSplit bwd16_split(int B, int H, int Hkv, int Sq, int Sk, int D, bool causal, bool masked, int cus) {
  BwdSplit sp;
  const int dk = bwd16_bucket(D);
  if (dk < 0 || (int64_t)B * H * Sq == 0 || Hkv < 1) return sp;
  const int occ_kv = dk <= 64 ? (causal ? 2 : 3) : dk <= 128 ? (masked && causal ? 1 : 2) : 1;
  const int occ_q = dk <= 64 ? (masked ? 2 : 3) : dk <= 128 ? (masked && causal ? 1 : 2) : 1;
  const int64_t n_kv = (int64_t)B * Hkv * ((Sk + 127) / 128), n_q = (int64_t)B * H * ((Sq + 127) / 128);
  const int64_t t_kv = (int64_t)(H / Hkv) * ((Sq + 31) / 32), t_q = (Sk + 31) / 32;
  sp.ns_kv = split_sweep(n_kv, occ_kv, cus, causal, t_kv);
  sp.ns_q = split_sweep(n_q, occ_q, cus, causal, t_q);
  // non-causal grids past one round: split only the last, partial round
  if (!causal && sp.ns_kv == 1) sp.ns_kv = split_tail(n_kv, occ_kv, cus, t_kv, &sp.nfull_kv);
  if (!causal && sp.ns_q == 1) sp.ns_q = split_tail(n_q, occ_q, cus, t_q, &sp.nfull_q);
  return sp;
}

hipError_t launch_bwd16(const BwdParams& p, bool bf16, bool causal, hipStream_t s) {
  if ((int64_t)p.B * p.H * p.Sq == 0) return hipSuccess;
  const int dk = bwd16_bucket(p.D);
  return bf16 ? launch_bwd_dtype<__bf16>(p, dk, causal, s) : launch_bwd_dtype<_Float16>(p, dk, causal, s);
}

}  // namespace cmpext3
