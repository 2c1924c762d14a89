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
  p.n_wg = p.B * p.Hkv * p.n_blk * ns;
  hipLaunchKernelGGL((attn_bwd_dkdv<T, DK, CAUSAL, MASK>), dim3(p.n_wg), dim3(256), 0, s, p);
  if (ns > 1) {
    const int64_t n4 = (int64_t)p.B * p.Hkv * p.Sk * p.D / 4;
    hipLaunchKernelGGL(attn_bwd_dkdv_reduce<T>, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s, p);
  }
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

// Workgroups of the dK/dV sweep per key block.  With too few key blocks for
// the CU slots the kernel's occupancy allows (one 4-wave workgroup per wave
// per SIMD), each block's sweep over (query head of the group, query tile)
// is cut into contiguous parts whose fp32 partials are summed afterwards:
// non-causal, as many parts as fill one round of slots; causal, enough for
// two rounds, so that the longest-first order evens out sweeps whose length
// falls with the key block (the first blocks see every query).  At most 8
// parts, each at least 4 query tiles of the longest sweep.
int bwd16_split(int B, int Hkv, int group, int Sq, int Sk, int D, bool causal, bool masked, int cus) {
  const int dk = bwd16_bucket(D);
  if (dk < 0 || (int64_t)B * Hkv * Sq == 0) return 1;
  const int occ = dk <= 64 ? (causal ? 2 : 3) : dk <= 128 ? (masked && causal ? 1 : 2) : 1;
  const int64_t n_wg = (int64_t)B * Hkv * ((Sk + 127) / 128);
  const int64_t slots = (int64_t)cus * occ;
  const int64_t want = causal ? 2 * slots : slots;
  if (n_wg * 2 > want) return 1;
  int64_t ns = causal ? (want + n_wg - 1) / n_wg : want / n_wg;
  const int64_t nj = (int64_t)group * ((Sq + 31) / 32);
  if (ns > 8) ns = 8;
  if (ns > nj / 4) ns = nj / 4;
  return ns >= 2 ? (int)ns : 1;
}

// Workspace of a split backward: fp32 partial dK and dV rows of every part.
size_t bwd_split_bytes(int B, int Hkv, int Sk, int D, int ns) {
  return ns > 1 ? (size_t)ns * B * Hkv * Sk * D * 2 * sizeof(float) : 0;
}

hipError_t launch_bwd16(const BwdParams& p, bool bf16, bool causal, hipStream_t s) {
  if ((int64_t)p.B * p.H * p.Sq == 0) return hipSuccess;
  const int dk = bwd16_bucket(p.D);
  return bf16 ? launch_bwd_dtype<__bf16>(p, dk, causal, s) : launch_bwd_dtype<_Float16>(p, dk, causal, s);
}

}  // namespace cmpext3
