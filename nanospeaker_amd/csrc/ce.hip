// Cross-entropy over the tied head's logits, one row per workgroup (16-bit types).
//
// Reference: NanoSpeaker.forward with targets (src/model/nanospeaker.py:236-250): the
// next-token loss F.cross_entropy((h @ embed.weight.T).float(), y), mean over the targets
// that are not ignore_index, with the logits rounded to the model's dtype by the GEMM.  The
// reference fuses the head and the loss on CUDA (LigerFusedLinearCrossEntropyLoss); here
// the two GEMMs stay library GEMMs (the host side, moe_kernel.linear_cross_entropy) and this
// kernel is the part between them:
//
//   ce_rows_kernel   reads a logits row once (V 16-bit values, held in registers: V / 256
//                    per thread), reduces its maximum and sum of exponentials in fp32 over
//                    the workgroup, and writes loss[row] = lse - logit[target] (0 for an
//                    ignored row).  With `grad` set it overwrites the row (in place is
//                    allowed) with d(mean loss) / d(logits) = (softmax - onehot(target)) / n
//                    rounded to the dtype, n = the number of targets that count, read from
//                    device memory so the host never waits for it; an ignored row's
//                    gradient is zero.  A target outside [0, V) that is not ignore_index
//                    gives a NaN loss (and is never read).
//
// A row is read once and written once: 4 bytes per logit of HBM traffic with the gradient,
// 2 without.
#include "../../include/nsmoe.h"
#include "gemm_core.h"
#include "nsmoe_capi_internal.h"

namespace nsmoe {

constexpr int CE_NT = 256;

template <int DT, int VPT>  // VPT: 16-byte vectors (8 elements) per thread
__global__ void __launch_bounds__(CE_NT) ce_rows_kernel(const uint16_t* logits, int64_t ld,
                                                        const int64_t* target, int64_t ignore,
                                                        const int64_t* n_valid, int V,
                                                        float* loss, uint16_t* grad) {
  __shared__ float s_red[CE_NT / 64];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint16_t* src = logits + row * ld;
  // Vector v of this thread covers elements (v * CE_NT + tid) * 8 .. + 7 (coalesced).
  u32x4 x[VPT];
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    const int e0 = (v * CE_NT + tid) * 8;
    x[v] = e0 < V ? *(const u32x4*)(src + e0) : u32x4{0u, 0u, 0u, 0u};
  }
  // The target's logit, read before any thread can overwrite the row with its gradient.
  // A target outside [0, V) that is not ignore_index gives a NaN loss (F.cross_entropy
  // raises there; a kernel cannot, and must not read outside the row).
  const int64_t y = target[row];
  const bool counted = y != ignore;
  const bool in_range = y >= 0 && y < V;
  float ylogit = 0.0f;
  if (tid == 0 && counted && in_range) ylogit = Elem<DT>::to_f(src[y]);
  auto block_reduce = [&](float val, bool is_max) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float other = __shfl_xor(val, o);
      val = is_max ? fmaxf(val, other) : val + other;
    }
    __syncthreads();  // s_red free from the previous reduction
    if (lane == 0) s_red[wave] = val;
    __syncthreads();
    float r = s_red[0];
#pragma unroll
    for (int w = 1; w < CE_NT / 64; ++w) r = is_max ? fmaxf(r, s_red[w]) : r + s_red[w];
    return r;
  };
  float mx = -INFINITY;
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    if ((v * CE_NT + tid) * 8 >= V) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, unpack2<DT>(x[v][e >> 1], e & 1));
  }
  mx = block_reduce(mx, true);
  constexpr float kLog2e = 1.4426950408889634f;
  const float mlog = mx * kLog2e;
  float sum = 0.0f;
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    if ((v * CE_NT + tid) * 8 >= V) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      sum += __builtin_amdgcn_exp2f(unpack2<DT>(x[v][e >> 1], e & 1) * kLog2e - mlog);
  }
  sum = block_reduce(sum, false);
  const float lse = mx + logf(sum);
  if (tid == 0) loss[row] = !counted ? 0.0f : in_range ? lse - ylogit : NAN;
  if (!grad) return;
  const int64_t nv = *n_valid;
  const float scale = counted && nv > 0 ? 1.0f / (float)nv : 0.0f;
  const float lse_log = lse * kLog2e;
  uint16_t* dst = grad + row * ld;
#pragma unroll
  for (int v = 0; v < VPT; ++v) {
    const int e0 = (v * CE_NT + tid) * 8;
    if (e0 >= V) continue;
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float g2[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int e = 2 * q + h;
        const float p = __builtin_amdgcn_exp2f(unpack2<DT>(x[v][q], h) * kLog2e - lse_log);
        g2[h] = (p - (e0 + e == y ? 1.0f : 0.0f)) * scale;
      }
      o[q] = pack2<DT>(g2[0], g2[1]);
    }
    *(u32x4*)(dst + e0) = o;
  }
}

template <int DT>
static int ce_launch(const uint16_t* logits, int64_t ld, int64_t n, int V, const int64_t* target,
                     int64_t ignore, const int64_t* n_valid, float* loss, uint16_t* grad,
                     hipStream_t s) {
  const int vpt = (int)cdiv(V, CE_NT * 8);
  KernelTimer timer("ce_rows", s);
  const unsigned grid = (unsigned)n;
#define NSMOE_CE(N)                                                                       \
  case N:                                                                                 \
    ce_rows_kernel<DT, N><<<grid, CE_NT, 0, s>>>(logits, ld, target, ignore, n_valid, V, \
                                                 loss, grad);                             \
    break;
  switch (vpt <= 4 ? 4 : vpt <= 8 ? 8 : vpt <= 16 ? 16 : 32) {
    NSMOE_CE(4) NSMOE_CE(8) NSMOE_CE(16) NSMOE_CE(32)
  }
#undef NSMOE_CE
  timer.stop();
  return check_launch("ce_rows_kernel");
}

}  // namespace nsmoe

using namespace nsmoe;

extern "C" int nsmoe_cross_entropy_rows(int32_t dtype, const void* logits, int64_t ld,
                                        int64_t n_rows, int32_t vocab, const int64_t* target,
                                        int64_t ignore_index, const int64_t* n_valid,
                                        float* loss, void* grad, void* stream) {
  NSMOE_REQUIRE(dtype == DT_BF16 || dtype == DT_F16, "cross_entropy: 16-bit types only");
  NSMOE_REQUIRE(n_rows >= 0 && n_rows < INT32_MAX, "cross_entropy: n_rows %lld out of range",
                (long long)n_rows);
  NSMOE_REQUIRE(vocab >= 1 && vocab % 8 == 0 && vocab <= CE_NT * 8 * 32,
                "cross_entropy: vocab %d must be a multiple of 8 and at most %d", vocab,
                CE_NT * 8 * 32);
  NSMOE_REQUIRE(ld >= vocab && ld % 8 == 0, "cross_entropy: row pitch %lld (need >= vocab, a "
                "multiple of 8)", (long long)ld);
  if (n_rows == 0) return NSMOE_OK;
  NSMOE_REQUIRE(logits && target && loss && (!grad || n_valid), "cross_entropy: NULL pointer");
  NSMOE_REQUIRE(((uintptr_t)logits & 15) == 0 && ((uintptr_t)grad & 15) == 0,
                "cross_entropy: logits and grad must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  return dtype == DT_BF16
             ? ce_launch<DT_BF16>((const uint16_t*)logits, ld, n_rows, vocab, target,
                                  ignore_index, n_valid, loss, (uint16_t*)grad, s)
             : ce_launch<DT_F16>((const uint16_t*)logits, ld, n_rows, vocab, target,
                                 ignore_index, n_valid, loss, (uint16_t*)grad, s);
}
