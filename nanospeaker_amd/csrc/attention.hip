// Prefill self-attention of the decoder around the MoE block (16-bit types, head dim 64).
//
// Reference: OptimizedMultiHeadAttention.forward on its SDPA path (src/model/mha.py:245-287,
// the band of causal_mask, mha.py:49-66): per-head RMSNorm of Q and K (qk_norm=True,
// F.rms_norm, src/model/ln.py:30-36), the rotary embedding (src/model/rope.py, rotate-half
// pairing over the whole head, tables cos/sin(pos * base^(-2j / d_head)) cast to the
// compute dtype, the rotation done in that dtype), causal attention in which query i sees
// key j when j <= i and, with a window w, i - j < w (the query counted), and grouped-query
// heads (query head h reads key/value head h / (Hq / Hkv)).
//
// Input is the fused projection qkv = Z [W_q | W_k | W_v]: each token's row holds Hq query
// heads, then Hkv key heads, then Hkv value heads, 64 elements each.
//
//   attn_k_prep_kernel  normalises and rotates the key heads in place (4 lanes per head
//                       row: lane j holds dims 8j .. 8j + 7 and their rotation partners
//                       32 + 8j .. 32 + 8j + 7, so the pairs are lane-local and the sum of
//                       squares needs two shuffles);
//   attn_fwd_kernel     one workgroup per (sequence, key/value head, 64 queries) with the
//                       G query heads of the group: 4 waves x G column blocks of 16
//                       (head, query) columns.  Each wave loads its queries straight into
//                       MFMA B fragments, normalising and rotating them in registers.  Key
//                       and value tiles of 64 rows are copied global -> LDS by LDS-DMA
//                       (three stages: two tiles in flight, one barrier per tile), with a
//                       chunk swizzle that keeps the fragment reads free of bank conflicts.
//
// The kernel computes S^T = K Q^T, so lane l of a wave ends with 4 consecutive keys of one
// query column (the MFMA accumulator layout).  Everything the online softmax needs per
// query is then in one lane or across the 4 lanes l, l ^ 16, l ^ 32, l ^ 48: the running
// maximum takes two lane swaps per tile, and the running sum comes from one more MFMA per
// P V step (a block of ones against P^T).  The probabilities are already the B operand of
// O^T = V^T P^T: for the 32 keys of a P V step, k slot 8 g + e (lane group g) is key
// 4 g + e of the first 16-key block and slot 8 g + 4 + e key 4 g + e of the second -- the
// keys the lane holds -- and
// the value rows are read in the same order with ds_read_b64_tr_b16.  No LDS round trip
// and no lane shuffles between the two GEMMs.
//
// Scores are scaled by log2(e) / sqrt(64) in fp32 and exponentiated with exp2; the
// probabilities enter the P V MFMA rounded to the dtype, their sums are accumulated in fp32
// over the same rounded values, and the output is divided by the sum and rounded once.
#include "../../include/nsmoe.h"
#include "gemm_core.h"
#include "nsmoe_capi_internal.h"

namespace nsmoe {

constexpr int AT_DH = 64;    // head dim
constexpr int AT_BQ = 64;    // queries per workgroup
constexpr int AT_BK = 64;    // keys per tile
constexpr int AT_NT = 256;   // threads per workgroup
constexpr int AT_TILE = AT_BK * AT_DH * 2;  // bytes of one K or V tile (16-bit)
constexpr int AT_STAGES = 3;                // K / V ring stages: two tiles in flight

struct AttnParams {
  uint16_t* qkv;           // [B * T, ld]
  uint16_t* out;           // [B * T, Hq * 64]
  const float* cosb;       // [T, 32] fp32
  const float* sinb;       // [T, 32] fp32
  const uint16_t* q_gamma; // [64]
  const uint16_t* k_gamma; // [64]
  int64_t B, T;
  int Hq, Hkv, ld, window;  // window: keys a query sees, itself included; 0 = all earlier
  float eps, scale_log2;
};

// Chunk swizzle of a 64-row x 128-byte tile: chunk c of row r sits at slot c ^ at_swz(r).
// A 16-byte fragment read (16 rows, one chunk) and a transposed read (8 rows x 32 bytes
// per 32 lanes) both land on distinct banks.
__device__ __forceinline__ int at_swz(int r) { return (((r >> 1) & 3) << 1) | ((r >> 3) & 1); }

// Maximum over lanes l, l ^ 16, l ^ 32, l ^ 48, in every lane.  v_permlane16_swap applied
// to two copies of v leaves v[l] in one result and v[l ^ 16] in the other (it exchanges
// the odd 16-lane rows of the first operand with the even rows of the second);
// v_permlane32_swap does the same for l ^ 32 with the two 32-lane halves.
__device__ __forceinline__ float max_xor16_32(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v),
                                                  false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// RMSNorm (F.rms_norm: fp32 rstd = 1 / sqrt(mean(x^2) + eps), x rstd gamma rounded once)
// and the rotation (in the dtype, as the reference's bf16 tensor ops: every product, the
// difference and the sum rounded) of one 64-element head row spread over 4 lanes: this
// lane holds dims 8 j .. 8 j + 7 in lo and 32 + 8 j .. 32 + 8 j + 7 in hi; `xor_a` and
// `xor_b` are the shuffle distances to the row's other three lanes.
template <int DT>
__device__ __forceinline__ void norm_rope_row(u32x4& lo, u32x4& hi, int j, int pos, bool live,
                                              const uint16_t* gamma, const float* cosb,
                                              const float* sinb, float eps, int xor_a,
                                              int xor_b) {
  float a[8], b[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = unpack2<DT>(lo[e >> 1], e & 1);
    b[e] = unpack2<DT>(hi[e >> 1], e & 1);
  }
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += a[e] * a[e] + b[e] * b[e];
  ss += __shfl_xor(ss, xor_a);
  ss += __shfl_xor(ss, xor_b);
  if (!live) return;
  const float rstd = 1.0f / sqrtf(ss / (float)AT_DH + eps);
  const u32x4 ga = *(const u32x4*)(gamma + 8 * j), gb = *(const u32x4*)(gamma + 32 + 8 * j);
  const float4* cp = (const float4*)(cosb + (int64_t)pos * (AT_DH / 2) + 8 * j);
  const float4* sp = (const float4*)(sinb + (int64_t)pos * (AT_DH / 2) + 8 * j);
  const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
  const float cs[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  // Every rounding to the dtype: bf16 goes two values at a time through the hardware's
  // packed round-to-nearest-even conversion (pack2) and back (the scalar software rounding
  // made this prologue a third of a windowed layer's time); fp16 rounds one value per
  // conversion instruction.  The last rounding of each output is the pack itself.
  auto rd2 = [](float& x, float& y) {
    if constexpr (DT == DT_BF16) {
      const uint32_t u = pack2<DT>(x, y);
      x = unpack2<DT>(u, 0);
      y = unpack2<DT>(u, 1);
    } else {
      x = Elem<DT>::to_f(Elem<DT>::from_f(x));
      y = Elem<DT>::to_f(Elem<DT>::from_f(y));
    }
  };
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = 2 * q;
    float x1a = a[e] * rstd * unpack2<DT>(ga[q], 0), x1b = a[e + 1] * rstd * unpack2<DT>(ga[q], 1);
    float x2a = b[e] * rstd * unpack2<DT>(gb[q], 0), x2b = b[e + 1] * rstd * unpack2<DT>(gb[q], 1);
    float ca = cs[e], cb = cs[e + 1], sa = sn[e], sb = sn[e + 1];
    rd2(x1a, x1b);
    rd2(x2a, x2b);
    rd2(ca, cb);
    rd2(sa, sb);
    float p1a = x1a * ca, p1b = x1b * cb, p2a = x2a * sa, p2b = x2b * sb;  // x1 c, x2 s
    float p3a = x2a * ca, p3b = x2b * cb, p4a = x1a * sa, p4b = x1b * sb;  // x2 c, x1 s
    rd2(p1a, p1b);
    rd2(p2a, p2b);
    rd2(p3a, p3b);
    rd2(p4a, p4b);
    const float d1a = p1a - p2a, d1b = p1b - p2b, d2a = p3a + p4a, d2b = p3b + p4b;
    if constexpr (DT == DT_BF16) {
      lo[q] = pack2<DT>(d1a, d1b);
      hi[q] = pack2<DT>(d2a, d2b);
    } else {
      lo[q] = (uint32_t)Elem<DT>::from_f(d1a) | ((uint32_t)Elem<DT>::from_f(d1b) << 16);
      hi[q] = (uint32_t)Elem<DT>::from_f(d2a) | ((uint32_t)Elem<DT>::from_f(d2b) << 16);
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(AT_NT) attn_k_prep_kernel(AttnParams p) {
  // 4 lanes per (token, key head) row, 64 rows per workgroup.
  const int64_t rows = p.B * p.T * p.Hkv;
  const int64_t r = (int64_t)blockIdx.x * (AT_NT / 4) + (threadIdx.x >> 2);
  const int j = threadIdx.x & 3;
  const bool live = r < rows;
  const int64_t rr = live ? r : 0;
  const int64_t tok = rr / p.Hkv;
  const int hk = (int)(rr % p.Hkv);
  const int pos = (int)(tok % p.T);
  uint16_t* row = p.qkv + tok * p.ld + (int64_t)(p.Hq + hk) * AT_DH;
  u32x4 lo = *(const u32x4*)(row + 8 * j), hi = *(const u32x4*)(row + 32 + 8 * j);
  norm_rope_row<DT>(lo, hi, j, pos, live, p.k_gamma, p.cosb, p.sinb, p.eps, 1, 2);
  if (live) {
    *(u32x4*)(row + 8 * j) = lo;
    *(u32x4*)(row + 32 + 8 * j) = hi;
  }
}

template <int DT, int G>
__global__ void __launch_bounds__(AT_NT, 2) attn_fwd_kernel(AttnParams p) {
  using M = Mma<DT>;
  using Frag = typename M::Frag;
  constexpr int NB = G;  // column blocks of 16 (head, query) columns per wave
  __shared__ __attribute__((aligned(1024))) char s_kv[AT_STAGES][2][AT_TILE];  // [stage][K, V]

  const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int T = (int)p.T;
  const int nqb = (T + AT_BQ - 1) / AT_BQ;
  const int pairs = (int)p.B * p.Hkv;
  const bool banded = p.window > 0 && p.window < T;
  int qb, pair;
  if (banded) {
    // Each XCD takes a contiguous run of query blocks: neighbouring blocks of one head
    // share all but one of their key tiles, so those stay in the XCD's L2.
    const int item = xcd_remap((int)blockIdx.x, (int)gridDim.x);
    pair = item / nqb;
    qb = item % nqb;
  } else {
    // Full causal: block qb reads qb + 1 tiles, so the longest go first.
    qb = nqb - 1 - (int)blockIdx.x / pairs;
    pair = (int)blockIdx.x % pairs;
  }
  const int b = pair / p.Hkv, hk = pair % p.Hkv;
  const int q0 = qb * AT_BQ;
  const int64_t row0 = (int64_t)b * T;
  const int qmax = min(q0 + AT_BQ - 1, T - 1);
  const int kmin = banded ? max(0, q0 - p.window + 1) : 0;
  const int t_first = kmin / AT_BK, t_last = qmax / AT_BK;
  const int64_t ld = p.ld;

  // The queries: this lane's column of block nb is query qpos[nb] of head hk G + gi.
  Frag qf[NB][2];
  int qpos[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int cb = wave * NB + nb;
    const int gi = cb >> 2;
    const int qp = q0 + 16 * (cb & 3) + l16;
    qpos[nb] = qp;
    const bool live = qp < T;
    u32x4 lo = {0u, 0u, 0u, 0u}, hi = {0u, 0u, 0u, 0u};
    if (live) {
      const uint16_t* src = p.qkv + (row0 + qp) * ld + (int64_t)(hk * G + gi) * AT_DH;
      lo = *(const u32x4*)(src + 8 * g);
      hi = *(const u32x4*)(src + 32 + 8 * g);
    }
    norm_rope_row<DT>(lo, hi, g, live ? qp : 0, live, p.q_gamma, p.cosb, p.sinb, p.eps, 16,
                      32);
    qf[nb][0].v = lo;
    qf[nb][1].v = hi;
  }
  // S^T k step ks contracts dims 32 ks .. 32 ks + 31: lane group g's 8 elements are dims
  // 32 ks + 8 g .. + 7, which is what lo (ks = 0) and hi (ks = 1) hold.

  // LDS-DMA copy plan: a tile is 8 K + 8 V copies of 1 KiB (8 rows x 128 bytes); wave w
  // issues copies 4 w .. 4 w + 3.  Lane i of a copy fills slot i % 8 of row i / 8 with
  // the global chunk (i % 8) ^ at_swz(row).
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)&s_kv[0][0][0];
  const uint16_t* zero = (const uint16_t*)((const char*)g_zero_kib + lane * 16);
  // Each copy's source for tile 0 is fixed per lane; tile t adds t * 64 rows (a
  // wave-uniform byte offset), and only a tile that runs past T checks its rows.
  const uint16_t* csrc[4];
  int crow[4];
  uint32_t cdst[4];
#pragma unroll
  for (int u4 = 0; u4 < 4; ++u4) {
    const int u = wave * 4 + u4;
    const int which = u >> 3, rb = u & 7;
    const int r = rb * 8 + (lane >> 3);
    const int c = (lane & 7) ^ at_swz(r);
    crow[u4] = r;
    csrc[u4] = p.qkv + (row0 + r) * ld + (int64_t)(p.Hq + which * p.Hkv + hk) * AT_DH + c * 8;
    cdst[u4] = lds0 + (uint32_t)(which * AT_TILE + rb * 1024);
  }
  const int64_t tile_step = (int64_t)AT_BK * ld;  // elements between tiles
  auto issue = [&](int t, int stage) {
    const int key0 = t * AT_BK;
    const int64_t off = (int64_t)t * tile_step;
    const bool whole = key0 + AT_BK <= T;  // uniform
#pragma unroll
    for (int u4 = 0; u4 < 4; ++u4) {
      const uint16_t* src = csrc[u4] + off;
      if (!whole && key0 + crow[u4] >= T) src = zero;
      async_copy16_to(src, cdst[u4] + (uint32_t)(stage * 2 * AT_TILE));
    }
  };

  // o[0..3]: O^T's four 16-dim blocks of each column block; o[4]: the row sums of the
  // probabilities, from one more MFMA per P V step against a block of ones (every lane
  // then holds its query's sum of the same rounded p the P V MFMAs used; no VALU adds
  // and no cross-lane reduction).
  f32x4 o[5][NB];
  float m[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    m[nb] = -INFINITY;
#pragma unroll
    for (int db = 0; db < 5; ++db) o[db][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  constexpr uint32_t one2 = DT == DT_BF16 ? 0x3F803F80u : 0x3C003C00u;  // two 1.0s
  const Frag ones{u32x4{one2, one2, one2, one2}};

  // Tiles t + 1 and t + 2 are in flight while tile t is computed: tile t + 2's copies go
  // into the stage tile t - 1 used, after the barrier that every wave reaches only once
  // done with tile t - 1.
  issue(t_first, 0);
  if (t_first < t_last) issue(t_first + 1, 1);
  for (int t = t_first; t <= t_last; ++t) {
    const int st = (t - t_first) % AT_STAGES;
    // this wave's copies of tile t (tile t + 1's four may stay in flight)
    if (t < t_last) wait_vmcnt<4>();
    else wait_vmcnt<0>();
    barrier_dma();    // every wave's copies of tile t; every wave done with tile t - 1
    if (t + 2 <= t_last) issue(t + 2, (st + 2) % AT_STAGES);
    const char* Kt = s_kv[st][0];
    const char* Vt = s_kv[st][1];
    const int key0 = t * AT_BK;

    // S^T = K Q^T over the 64 dims: s[kb][nb] holds keys key0 + 16 kb + 4 g + e of this
    // lane's query column.
    f32x4 s[4][NB];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s[kb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        const int r = 16 * kb + l16, c = 4 * ks + g;
        const Frag kf = M::load(Kt + r * 128 + ((c ^ at_swz(r)) << 4));
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) M::run(s[kb][nb], kf, qf[nb][ks]);
      }
    }

    // Mask, only on tiles that cross the diagonal or the window's far edge: one uniform
    // branch, then a select per score (no per-score control flow).
    const bool masked = key0 + AT_BK - 1 > q0 || (banded && key0 < qmax - p.window + 1);
    if (masked) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int q = qpos[nb];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int key = key0 + 16 * kb + 4 * g + e;
            const bool dead = (key > q) | (banded & (q - key >= p.window));
            s[kb][nb][e] = dead ? -INFINITY : s[kb][nb][e];
          }
      }
    }
    // Online softmax.  The running maximum m is kept on the raw scores; p = 2^(s c - m c)
    // with c = log2(e) / 8 is one FMA and one exp2 per score.  A query's 16 scores of the
    // tile sit in lanes l, l ^ 16, l ^ 32, l ^ 48: their maximum takes two lane swaps
    // (v_permlane16_swap / v_permlane32_swap, VALU, no LDS round trip).
    const float c = p.scale_log2;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      // The tile's maximum (m[nb] enters the max3 chain: it is equal in the query's 4
      // lanes).
      float mx = m[nb];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) mx = fmaxf(mx, s[kb][nb][e]);
      mx = max_xor16_32(mx);
      // Lazy rescaling: m[nb] is the reference the exponents are taken against, moved
      // (with the accumulators rescaled by 2^((m_old - m_new) c)) only when some query's
      // scores would exceed it by more than 2^8 -- or on its first finite score.  p stays
      // <= 256, well inside the 16-bit and fp32 ranges, and the output is the same ratio
      // sum p v / sum p whatever the reference; the wave-uniform branch is rarely taken
      // once the first tiles have set the scale.
      const bool move = m[nb] == -INFINITY ? mx != -INFINITY : (mx - m[nb]) * c > 8.0f;
      if (__ballot(move)) {
        const float mnew = move ? mx : m[nb];
        const float alpha = m[nb] == -INFINITY ? 0.0f
                                               : __builtin_amdgcn_exp2f((m[nb] - mnew) * c);
#pragma unroll
        for (int db = 0; db < 5; ++db) o[db][nb] *= alpha;
        m[nb] = mnew;
      }
      const float msub = m[nb] == -INFINITY ? 0.0f : m[nb] * c;  // no key seen yet: p = 0
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          s[kb][nb][e] = __builtin_amdgcn_exp2f(fmaf(s[kb][nb][e], c, -msub));
    }

    // O^T += V^T P^T over the 64 keys, 32 at a time (key blocks 2 ks and 2 ks + 1).
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      Frag pf[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 a = s[2 * ks][nb], c = s[2 * ks + 1][nb];
        pf[nb].v = u32x4{pack2<DT>(a[0], a[1]), pack2<DT>(a[2], a[3]), pack2<DT>(c[0], c[1]),
                         pack2<DT>(c[2], c[3])};
      }
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int i = l16;
        const int ra = 32 * ks + 4 * g + (i >> 2), rb = ra + 16;
        const int cc = 2 * db + ((i & 3) >> 1), within = 8 * (i & 1);
        const uint2 lo = lds_read_tr16(Vt + ra * 128 + ((cc ^ at_swz(ra)) << 4) + within);
        const uint2 hi = lds_read_tr16(Vt + rb * 128 + ((cc ^ at_swz(rb)) << 4) + within);
        Frag vf;
        vf.v = u32x4{lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) M::run(o[db][nb], vf, pf[nb]);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) M::run(o[4][nb], ones, pf[nb]);
    }
  }

  // O / sum, rounded once: lane holds dims 16 db + 4 g .. + 3 of its query column.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float l = o[4][nb][0];
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    const int qp = qpos[nb];
    if (qp >= T) continue;
    const int gi = (wave * NB + nb) >> 2;
    uint16_t* dst = p.out + (row0 + qp) * (int64_t)(p.Hq * AT_DH) + (int64_t)(hk * G + gi) * AT_DH +
                    4 * g;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const f32x4 v = o[db][nb] * inv;
      *(uint2*)(dst + 16 * db) = make_uint2(pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]));
    }
  }
}

template <int DT>
static int attn_launch(const AttnParams& P, int G, hipStream_t s) {
  const int64_t krows = P.B * P.T * P.Hkv;
  const unsigned gk = (unsigned)cdiv(krows, AT_NT / 4);
  const int64_t nqb = cdiv(P.T, AT_BQ);
  const int64_t grid = nqb * P.B * P.Hkv;
  NSMOE_REQUIRE(grid < INT32_MAX && gk < INT32_MAX, "attn_prefill: grid too large");
  {
    KernelTimer timer("attn_k_prep", s);
    attn_k_prep_kernel<DT><<<gk, AT_NT, 0, s>>>(P);
    timer.stop();
  }
  NSMOE_TRY(check_launch("attn_k_prep_kernel"));
  KernelTimer timer("attn_fwd", s);
  switch (G) {
    case 1: attn_fwd_kernel<DT, 1><<<(unsigned)grid, AT_NT, 0, s>>>(P); break;
    case 2: attn_fwd_kernel<DT, 2><<<(unsigned)grid, AT_NT, 0, s>>>(P); break;
    case 3: attn_fwd_kernel<DT, 3><<<(unsigned)grid, AT_NT, 0, s>>>(P); break;
    default: attn_fwd_kernel<DT, 4><<<(unsigned)grid, AT_NT, 0, s>>>(P); break;
  }
  timer.stop();
  return check_launch("attn_fwd_kernel");
}

}  // namespace nsmoe

using namespace nsmoe;

extern "C" int nsmoe_attn_prefill(const nsmoe_attn_args* a, void* stream) {
  NSMOE_REQUIRE(a, "attn_prefill: NULL args");
  NSMOE_REQUIRE(a->dtype == DT_BF16 || a->dtype == DT_F16, "attn_prefill: 16-bit types only");
  NSMOE_REQUIRE(a->head_dim == AT_DH, "attn_prefill: head_dim must be 64 (got %d)", a->head_dim);
  NSMOE_REQUIRE(a->n_kv_heads >= 1 && a->n_heads >= a->n_kv_heads &&
                    a->n_heads % a->n_kv_heads == 0 && a->n_heads / a->n_kv_heads <= 4,
                "attn_prefill: n_heads %d must be 1-4 times n_kv_heads %d", a->n_heads,
                a->n_kv_heads);
  NSMOE_REQUIRE(a->batch >= 0 && a->seq_len >= 0 && a->seq_len < (1 << 30),
                "attn_prefill: bad batch / seq_len");
  NSMOE_REQUIRE(a->window >= 0, "attn_prefill: window %d < 0", a->window);
  NSMOE_REQUIRE(a->ld >= (a->n_heads + 2 * a->n_kv_heads) * AT_DH && a->ld % 8 == 0,
                "attn_prefill: qkv pitch %d (need >= %d, a multiple of 8)", a->ld,
                (a->n_heads + 2 * a->n_kv_heads) * AT_DH);
  if (a->batch == 0 || a->seq_len == 0) return NSMOE_OK;
  NSMOE_REQUIRE(a->qkv && a->out && a->q_gamma && a->k_gamma && a->cos && a->sin,
                "attn_prefill: NULL pointer");
  NSMOE_REQUIRE(((uintptr_t)a->qkv & 15) == 0 && ((uintptr_t)a->out & 7) == 0 &&
                    ((uintptr_t)a->q_gamma & 15) == 0 && ((uintptr_t)a->k_gamma & 15) == 0 &&
                    ((uintptr_t)a->cos & 15) == 0 && ((uintptr_t)a->sin & 15) == 0,
                "attn_prefill: misaligned pointer");
  AttnParams P{};
  P.qkv = (uint16_t*)a->qkv;
  P.out = (uint16_t*)a->out;
  P.cosb = a->cos;
  P.sinb = a->sin;
  P.q_gamma = (const uint16_t*)a->q_gamma;
  P.k_gamma = (const uint16_t*)a->k_gamma;
  P.B = a->batch;
  P.T = a->seq_len;
  P.Hq = a->n_heads;
  P.Hkv = a->n_kv_heads;
  P.ld = a->ld;
  P.window = a->window;
  P.eps = a->eps;
  P.scale_log2 = 1.4426950408889634f / 8.0f;  // log2(e) / sqrt(64)
  const int G = a->n_heads / a->n_kv_heads;
  hipStream_t s = (hipStream_t)stream;
  return a->dtype == DT_BF16 ? attn_launch<DT_BF16>(P, G, s) : attn_launch<DT_F16>(P, G, s);
}
