// The RMSNorm in front of the block and the residual around it, backward (16-bit types).
//
// Reference: Block.forward's FFN half, x + ffn(norm_ffn(x)) (src/model/nanospeaker.py:169),
// with norm_ffn an RMSNorm (src/model/ln.py:30-36, F.rms_norm).  Its forward is fused into
// the block's other kernels: the router kernel normalises the rows it loads for the
// router GEMM and stores them for the experts (router.hip), and the combine adds the
// residual (experts.hip).  The backward, given the block's input gradient dxn (the
// combine of the expert dX rows and the router term, rounded to the dtype):
//
//   norm_bwd_kernel     per token row, F.rms_norm's backward in fp32,
//                         xh = x rstd,  gxh = dxn w,  s = sum_c xh gxh,
//                         dx_norm = (gxh - (xh / d) s) rstd      (rounded to the dtype)
//                       plus the residual's gradient: dx = g + dx_norm (rounded again), and
//                       this workgroup's fp32 column sums of dxn xh for the gain's gradient;
//   norm_dw_reduce      those partial sums added in workgroup order -> dw (the dtype).
#include "../../include/nsmoe.h"
#include "gemm_core.h"
#include "nsmoe_capi_internal.h"
#include "norm.h"

namespace nsmoe {

constexpr int NB_THREADS = 256;
constexpr int NB_MAXU = NORM_MAX_D / 8 / 64;  // 16-byte chunks per lane of a row

template <int DT>
__global__ void __launch_bounds__(NB_THREADS) norm_bwd_kernel(NormBwdArgs a) {
  using ET = typename Elem<DT>::T;
  __shared__ float s_part[NB_THREADS / 64][NORM_MAX_D];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int d = a.d, nch = d / 8;
  const float inv_d = 1.0f / (float)d;
  const int64_t r0 = (int64_t)blockIdx.x * NORM_ROWS;
  const int64_t r1 = min(r0 + NORM_ROWS, a.T);
  // The gain of this lane's chunks, and its column sums of dxn xh.
  float w[NB_MAXU][8], dw[NB_MAXU][8];
#pragma unroll
  for (int u = 0; u < NB_MAXU; ++u) {
    const int c = lane + 64 * u;
    u32x4 wv = u32x4{0u, 0u, 0u, 0u};
    if (c < nch) wv = *(const u32x4*)((const ET*)a.w + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      w[u][e] = unpack2<DT>(wv[e / 2], e & 1);
      dw[u][e] = 0.0f;
    }
  }
  for (int64_t t = r0 + wave; t < r1; t += NB_THREADS / 64) {  // uniform per wave
    const float rstd = a.rstd[t];
    float xh[NB_MAXU][8], gxh[NB_MAXU][8], g[NB_MAXU][8];
    float dot = 0.0f;
#pragma unroll
    for (int u = 0; u < NB_MAXU; ++u) {
      const int c = lane + 64 * u;
      u32x4 xv = u32x4{0u, 0u, 0u, 0u}, dv = xv, gv = xv;
      if (c < nch) {
        xv = *(const u32x4*)((const ET*)a.x + t * d + 8 * c);
        dv = *(const u32x4*)((const ET*)a.dxn + t * d + 8 * c);
        gv = *(const u32x4*)((const ET*)a.g + t * d + 8 * c);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float dn = unpack2<DT>(dv[e / 2], e & 1);
        xh[u][e] = unpack2<DT>(xv[e / 2], e & 1) * rstd;
        gxh[u][e] = dn * w[u][e];
        g[u][e] = unpack2<DT>(gv[e / 2], e & 1);
        dot += xh[u][e] * gxh[u][e];
        dw[u][e] += dn * xh[u][e];
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
#pragma unroll
    for (int u = 0; u < NB_MAXU; ++u) {
      const int c = lane + 64 * u;
      if (c >= nch) continue;
      u32x4 ov;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float v[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float dnorm = Elem<DT>::to_f(
              Elem<DT>::from_f((gxh[u][e + h] - (xh[u][e + h] * inv_d) * dot) * rstd));
          v[h] = g[u][e + h] + dnorm;
        }
        ov[e / 2] = pack2<DT>(v[0], v[1]);
      }
      *(u32x4*)((ET*)a.dx + t * d + 8 * c) = ov;
    }
  }
  // The workgroup's column sums: each wave's, then the 4 waves in order.
#pragma unroll
  for (int u = 0; u < NB_MAXU; ++u) {
    const int c = lane + 64 * u;
    if (c < nch) {
#pragma unroll
      for (int e = 0; e < 8; ++e) s_part[wave][8 * c + e] = dw[u][e];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += NB_THREADS) {
    float v = 0.0f;
#pragma unroll
    for (int q = 0; q < NB_THREADS / 64; ++q) v += s_part[q][c];
    a.partial[(int64_t)blockIdx.x * d + c] = v;
  }
}

template <int DT>
__global__ void __launch_bounds__(NB_THREADS) norm_dw_reduce_kernel(NormBwdArgs a, int nwg) {
  const int c = blockIdx.x * NB_THREADS + threadIdx.x;
  if (c >= a.d) return;
  float v = 0.0f;
  for (int q = 0; q < nwg; ++q) v += a.partial[(int64_t)q * a.d + c];
  ((typename Elem<DT>::T*)a.dw)[c] = Elem<DT>::from_f(v);
}

size_t norm_bwd_partial_bytes(int64_t T, int d) {
  return (size_t)((T + NORM_ROWS - 1) / NORM_ROWS) * (size_t)d * sizeof(float);
}

int norm_bwd_launch(int dtype, const NormBwdArgs& a, hipStream_t s) {
  NSMOE_REQUIRE(dtype == DT_BF16 || dtype == DT_F16, "norm_bwd: 16-bit types only");
  NSMOE_REQUIRE(a.d >= 8 && a.d % 8 == 0 && a.d <= NORM_MAX_D,
                "norm_bwd: d %% 8 == 0 and d <= %d (d %d)", NORM_MAX_D, a.d);
  NSMOE_REQUIRE(a.x && a.rstd && a.w && a.dxn && a.g && a.dx && a.partial && a.dw,
                "norm_bwd: NULL pointer");
  if (a.T == 0) return NSMOE_OK;
  const int nwg = (int)((a.T + NORM_ROWS - 1) / NORM_ROWS);
  const unsigned rg = (unsigned)((a.d + NB_THREADS - 1) / NB_THREADS);
  KernelTimer timer("norm_bwd", s);
  if (dtype == DT_BF16) {
    norm_bwd_kernel<DT_BF16><<<(unsigned)nwg, NB_THREADS, 0, s>>>(a);
    norm_dw_reduce_kernel<DT_BF16><<<rg, NB_THREADS, 0, s>>>(a, nwg);
  } else {
    norm_bwd_kernel<DT_F16><<<(unsigned)nwg, NB_THREADS, 0, s>>>(a);
    norm_dw_reduce_kernel<DT_F16><<<rg, NB_THREADS, 0, s>>>(a, nwg);
  }
  timer.stop();
  return check_launch("norm_bwd_kernel");
}

// ---- the forward, on its own ------------------------------------------------------------
//
// y = RMSNorm(x) for the norms the block's kernels do not take (the attention's pre-norm and
// the final norm of the decoder around the block): F.rms_norm's arithmetic, fp32
// rstd = 1 / sqrt(mean(x^2) + eps) and y = (x rstd) w rounded once, as the router kernel's
// fused norm computes it.  A wave takes NF_ROWS rows (16-byte chunks, two per lane at
// d <= 1024) and issues all their loads before the first sum of squares, so each wave keeps
// NF_ROWS rows in flight; each row's sum is a wave butterfly.  A row is one read and one
// write of HBM.
constexpr int NF_ROWS = 4;

template <int DT>
__global__ void __launch_bounds__(NB_THREADS) norm_fwd_kernel(const void* __restrict__ x,
                                                              const void* __restrict__ w,
                                                              void* __restrict__ y,
                                                              float* __restrict__ rstd_out,
                                                              int64_t T, int d, float eps) {
  using ET = typename Elem<DT>::T;
  const int lane = threadIdx.x & 63;
  const int64_t t0 = ((int64_t)blockIdx.x * (NB_THREADS / 64) + (threadIdx.x >> 6)) * NF_ROWS;
  if (t0 >= T) return;  // uniform per wave; no workgroup barrier below
  const int nch = d / 8;
  u32x4 xv[NF_ROWS][NB_MAXU];
#pragma unroll
  for (int r = 0; r < NF_ROWS; ++r)
#pragma unroll
    for (int u = 0; u < NB_MAXU; ++u) {
      const int c = lane + 64 * u;
      xv[r][u] = c < nch && t0 + r < T ? *(const u32x4*)((const ET*)x + (t0 + r) * d + 8 * c)
                                       : u32x4{0u, 0u, 0u, 0u};
    }
  u32x4 wv[NB_MAXU];
#pragma unroll
  for (int u = 0; u < NB_MAXU; ++u) {
    const int c = lane + 64 * u;
    wv[u] = c < nch ? *(const u32x4*)((const ET*)w + 8 * c) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int r = 0; r < NF_ROWS; ++r) {
    const int64_t t = t0 + r;
    if (t >= T) break;  // uniform
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < NB_MAXU; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = unpack2<DT>(xv[r][u][e / 2], e & 1);
        ss += v * v;
      }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float rstd = 1.0f / sqrtf(ss / (float)d + eps);
    if (rstd_out && lane == 0) rstd_out[t] = rstd;
#pragma unroll
    for (int u = 0; u < NB_MAXU; ++u) {
      const int c = lane + 64 * u;
      if (c >= nch) continue;
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        o[q] = pack2<DT>(unpack2<DT>(xv[r][u][q], 0) * rstd * unpack2<DT>(wv[u][q], 0),
                         unpack2<DT>(xv[r][u][q], 1) * rstd * unpack2<DT>(wv[u][q], 1));
      *(u32x4*)((ET*)y + t * d + 8 * c) = o;
    }
  }
}

}  // namespace nsmoe

using namespace nsmoe;

extern "C" int nsmoe_rms_norm(int32_t dtype, const void* x, const void* weight, float eps,
                              int64_t n_rows, int32_t d, void* y, float* rstd, void* stream) {
  NSMOE_REQUIRE(dtype == DT_BF16 || dtype == DT_F16, "rms_norm: 16-bit types only");
  NSMOE_REQUIRE(d >= 8 && d % 8 == 0 && d <= NORM_MAX_D,
                "rms_norm: d %% 8 == 0 and d <= %d (d %d)", NORM_MAX_D, d);
  NSMOE_REQUIRE(n_rows >= 0, "rms_norm: n_rows %lld < 0", (long long)n_rows);
  if (n_rows == 0) return NSMOE_OK;
  NSMOE_REQUIRE(x && weight && y, "rms_norm: NULL pointer");
  NSMOE_REQUIRE(((uintptr_t)x & 15) == 0 && ((uintptr_t)weight & 15) == 0 &&
                    ((uintptr_t)y & 15) == 0,
                "rms_norm: x, weight and y must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const int64_t rows_per_wg = (int64_t)(NB_THREADS / 64) * NF_ROWS;
  const int64_t grid = (n_rows + rows_per_wg - 1) / rows_per_wg;
  NSMOE_REQUIRE(grid < INT32_MAX, "rms_norm: too many rows");
  KernelTimer timer("norm_fwd", s);
  if (dtype == DT_BF16)
    norm_fwd_kernel<DT_BF16><<<(unsigned)grid, NB_THREADS, 0, s>>>(x, weight, y, rstd, n_rows, d, eps);
  else
    norm_fwd_kernel<DT_F16><<<(unsigned)grid, NB_THREADS, 0, s>>>(x, weight, y, rstd, n_rows, d, eps);
  timer.stop();
  return check_launch("norm_fwd_kernel");
}
