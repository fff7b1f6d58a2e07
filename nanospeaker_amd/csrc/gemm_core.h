// MFMA building blocks for the grouped expert GEMMs on gfx950.
//
// Operand tiles live in LDS "k-major": one row per output row (A) or output column (B),
// 32 contraction elements per row -- exactly one MFMA k-step -- padded by 16 bytes so
// the 16 lanes that read one 16x16 block's fragments hit distinct banks.
//
// MFMA contract used everywhere (v_mfma_f32_16x16x32_{bf16,f16}; fp32 issues eight
// v_mfma_f32_16x16x4_f32 over the same 32 elements):
//   A fragment: lane l supplies row (l % 16), k elements [8 * (l / 16), +8)
//   B fragment: lane l supplies column (l % 16), the same k elements
//   D:          lane l holds rows 4 * (l / 16) + {0..3} of column (l % 16)
// A and B always draw their k elements through the same (lane, slot) assignment, so the
// contraction does not depend on how the hardware orders k inside an instruction.
#pragma once

#include "nsmoe_common.h"

namespace nsmoe {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

template <int DT> struct Geo {
  using T = typename Elem<DT>::T;
  static constexpr int ES = (int)sizeof(T);  // element bytes: 2 or 4
  static constexpr int VE = 16 / ES;         // elements per 16-byte vector
  static constexpr int KC = 32;              // contraction elements per LDS row
  static constexpr int ROWB = KC * ES;       // 64 or 128 bytes
  static constexpr int PITCH = ROWB + 16;    // LDS row pitch (bytes)
  static constexpr int VPR = ROWB / 16;      // 16-byte vectors per LDS row
  static constexpr int FRAGB = 8 * ES;       // bytes one lane reads per fragment
};

template <int DT> struct Mma;

template <> struct Mma<DT_BF16> {
  struct Frag { u32x4 v; };
  __device__ static Frag load(const char* p) { return Frag{*(const u32x4*)p}; }
  __device__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.v),
                                                  __builtin_bit_cast(bf16x8, b.v), acc, 0, 0, 0);
  }
};

template <> struct Mma<DT_F16> {
  struct Frag { u32x4 v; };
  __device__ static Frag load(const char* p) { return Frag{*(const u32x4*)p}; }
  __device__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a.v),
                                                 __builtin_bit_cast(f16x8, b.v), acc, 0, 0, 0);
  }
};

template <> struct Mma<DT_F32> {
  struct Frag { u32x4 lo, hi; };
  __device__ static Frag load(const char* p) {
    return Frag{*(const u32x4*)p, *(const u32x4*)(p + 16)};
  }
  __device__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.lo[i]),
                                                 __uint_as_float(b.lo[i]), acc, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.hi[i]),
                                                 __uint_as_float(b.hi[i]), acc, 0, 0, 0);
  }
};

// Fragment of the 16-row block starting at `row0` of a k-major LDS tile.
template <int DT>
__device__ __forceinline__ typename Mma<DT>::Frag frag_at(const char* tile, int pitch,
                                                          int row0, int kbyte0) {
  const int l = lane_id();
  return Mma<DT>::load(tile + (row0 + (l & 15)) * pitch + kbyte0 + (l >> 4) * Geo<DT>::FRAGB);
}

__device__ __forceinline__ uint32_t lane_half(const u32x4& v, int c) {
  uint32_t d = v[c >> 1];
  return (c & 1) ? (d >> 16) : (d & 0xffffu);
}

// ---- staging: global -> registers -> LDS ---------------------------------------------
//
// DirectStage copies NROWS rows of 32 contraction elements whose source is contiguous in
// k (row r, element k at rowptr(r)[k]).  TransStage builds the same k-major tile from a
// source that is contiguous in the other index (element (k, n) at rowptr(k)[n]): each
// thread loads a VE x VE block with 16-byte loads and transposes it in registers.
// `fast` means every source vector is 16-byte aligned and either fully inside or fully
// outside the valid range; otherwise elements are loaded one by one.

template <int DT, int NROWS, int NT>
struct DirectStage {
  using G = Geo<DT>;
  using T = typename G::T;
  static constexpr int NV = NROWS * G::VPR;
  static constexpr int PER = (NV + NT - 1) / NT;
  u32x4 v[PER];

  // Source columns [k0, k0 + 32), valid below klim.
  template <class RowPtr>
  __device__ __forceinline__ void load(RowPtr rowptr, int k0, int klim, bool fast) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = threadIdx.x + i * NT;
      v[i] = u32x4{0u, 0u, 0u, 0u};
      if (NV % NT == 0 || idx < NV) {
        const int r = idx / G::VPR, c = idx % G::VPR;
        const T* src = rowptr(r);
        const int kk = k0 + c * G::VE;
        if (src) {
          if (fast) {
            if (kk < klim) v[i] = *(const u32x4*)(src + kk);
          } else {
            T tmp[G::VE];
#pragma unroll
            for (int e = 0; e < G::VE; ++e) tmp[e] = (kk + e < klim) ? src[kk + e] : T(0);
            __builtin_memcpy(&v[i], tmp, 16);
          }
        }
      }
    }
  }

  __device__ __forceinline__ void store(char* tile) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = threadIdx.x + i * NT;
      if (NV % NT == 0 || idx < NV) {
        const int r = idx / G::VPR, c = idx % G::VPR;
        *(u32x4*)(tile + r * G::PITCH + c * 16) = v[i];
      }
    }
  }
};

template <int DT, int NCOLS, int NT>
struct TransStage {
  using G = Geo<DT>;
  using T = typename G::T;
  static constexpr int KB = G::KC / G::VE;  // k blocks per chunk
  static constexpr int NB = NCOLS / G::VE;  // n blocks per tile
  static constexpr int NBLK = KB * NB;
  static constexpr int PER = (NBLK + NT - 1) / NT;
  u32x4 v[PER][G::VE];

  // Source rows k in [k0, k0 + 32) (valid below klim), columns [n0, n0 + NCOLS) (valid
  // below nlim).  scale(k) multiplies the row in fp32 before it is re-rounded; rows
  // whose rowptr is null load as zero.
  template <class RowPtr, class Scale>
  __device__ __forceinline__ void load(RowPtr rowptr, Scale scale, int k0, int klim, int n0,
                                       int nlim, bool fast) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = threadIdx.x + i * NT;
      const bool live = (NBLK % NT == 0) || blk < NBLK;
      const int kb = blk / NB, nb = blk % NB;
      const int col = n0 + nb * G::VE;
#pragma unroll
      for (int r = 0; r < G::VE; ++r) {
        v[i][r] = u32x4{0u, 0u, 0u, 0u};
        const int k = k0 + kb * G::VE + r;
        if (!live || k >= klim) continue;
        const T* src = rowptr(k);
        if (!src) continue;
        T tmp[G::VE];
        if (fast) {
          if (col < nlim) {
            u32x4 raw = *(const u32x4*)(src + col);
            __builtin_memcpy(tmp, &raw, 16);
          } else {
#pragma unroll
            for (int e = 0; e < G::VE; ++e) tmp[e] = T(0);
          }
        } else {
#pragma unroll
          for (int e = 0; e < G::VE; ++e) tmp[e] = (col + e < nlim) ? src[col + e] : T(0);
        }
        const float s = scale(k);
        if (s != 1.0f) {
#pragma unroll
          for (int e = 0; e < G::VE; ++e) tmp[e] = Elem<DT>::from_f(Elem<DT>::to_f(tmp[e]) * s);
        }
        __builtin_memcpy(&v[i][r], tmp, 16);
      }
    }
  }

  __device__ __forceinline__ void store(char* tile) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = threadIdx.x + i * NT;
      if (!((NBLK % NT == 0) || blk < NBLK)) continue;
      const int kb = blk / NB, nb = blk % NB;
      char* dst = tile + (nb * G::VE) * G::PITCH + kb * G::VE * G::ES;
      if constexpr (G::ES == 2) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          u32x4 o;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            o[q] = lane_half(v[i][2 * q], c) | (lane_half(v[i][2 * q + 1], c) << 16);
          *(u32x4*)(dst + c * G::PITCH) = o;
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4 o{v[i][0][c], v[i][1][c], v[i][2][c], v[i][3][c]};
          *(u32x4*)(dst + c * G::PITCH) = o;
        }
      }
    }
  }
};

struct NoScale {
  __device__ __forceinline__ float operator()(int) const { return 1.0f; }
};

// ---- tile scheduling over ragged groups -------------------------------------------------
//
// Groups are the routed experts (rows = their routing counts) followed by the shared
// experts (rows = every token).  `units(g)` says how many work items group g owns (for
// a GEMM: ceil(rows / BM)); locate() finds which group owns work item `item`, and the
// item's index inside that group.  Wave 0 scans the unit counts 64 groups at a time;
// the answer is broadcast through LDS.  Returns false past the last item.
struct Located {
  int g;
  int local;
  int aux;  // prefix of aux(g) over the groups before g
};

template <class Units, class Aux>
__device__ __forceinline__ bool locate(int item, int G, Units units, Aux aux, int* s_loc,
                                       Located& out) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int base = 0, abase = 0;
    int fg = -1, floc = 0, faux = 0;
    for (int g0 = 0; g0 < G; g0 += 64) {
      const int g = g0 + lane;
      const int u = g < G ? units(g) : 0;
      const int a = g < G ? aux(g) : 0;
      int incl = u, aincl = a;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        int t = __shfl_up(incl, o, 64);
        int ta = __shfl_up(aincl, o, 64);
        if (lane >= o) {
          incl += t;
          aincl += ta;
        }
      }
      const bool hit = item >= base + incl - u && item < base + incl;
      const unsigned long long m = __ballot(hit);
      if (m) {
        const int src = __ffsll((long long)m) - 1;
        const int excl = __shfl(incl - u, src, 64);
        const int aexcl = __shfl(aincl - a, src, 64);
        fg = g0 + src;
        floc = item - base - excl;
        faux = abase + aexcl;
        break;
      }
      base += __shfl(incl, 63, 64);
      abase += __shfl(aincl, 63, 64);
    }
    if (lane == 0) {
      s_loc[0] = fg;
      s_loc[1] = floc;
      s_loc[2] = faux;
    }
  }
  __syncthreads();
  out.g = s_loc[0];
  out.local = s_loc[1];
  out.aux = s_loc[2];
  return out.g >= 0;
}

// Consecutive work items (same expert, same weights) are placed on the same XCD: the
// dispatcher deals workgroup ids round-robin over the 8 XCDs, so id b runs on XCD b % 8.
__device__ __forceinline__ int xcd_remap(int bid, int grid) {
  const int q = grid / 8, rr = grid % 8;
  const int x = bid % 8, j = bid / 8;
  return x * q + (x < rr ? x : rr) + j;
}

}  // namespace nsmoe
