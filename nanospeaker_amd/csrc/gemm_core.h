// MFMA building blocks for the grouped expert GEMMs on gfx950.
//
// MFMA contract used everywhere (v_mfma_f32_16x16x32_{bf16,f16}; fp32 issues eight
// v_mfma_f32_16x16x4_f32 over the same 32 elements):
//   A fragment: lane l supplies row (l % 16), k elements [8 * (l / 16), +8)
//   B fragment: lane l supplies column (l % 16), the same k elements
//   D:          lane l holds rows 4 * (l / 16) + {0..3} of column (l % 16)
// A and B always draw their k elements through the same (lane, slot) assignment, so the
// contraction does not depend on how the hardware orders k inside an instruction.
//
// Operand placement:
//   * Weights reach the MFMAs straight from global memory (L2-resident).  Those whose
//     contraction index is not contiguous in memory (W_in for GEMM1, W_out for GEMM2)
//     are first repacked into "fragment order" (pack.hip): the 64 lanes' 16-byte pieces
//     of one 16 x 32 fragment are one contiguous 1 KiB block, so a fragment is a single
//     fully coalesced load.
//   * Token rows (the gathered A operand, shared by all waves of a workgroup) are staged
//     through LDS in 32-element rows with an XOR swizzle of the 16-byte chunks, so both
//     the staging stores and the 16-lane fragment reads touch distinct banks.
#pragma once

#include "nsmoe_common.h"

namespace nsmoe {

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

template <int DT> struct Geo {
  using T = typename Elem<DT>::T;
  static constexpr int ES = (int)sizeof(T);  // element bytes: 2 or 4
  static constexpr int VE = 16 / ES;         // elements per 16-byte vector
  static constexpr int KC = 32;              // contraction elements per LDS row
  static constexpr int ROWB = KC * ES;       // 64 or 128 bytes per LDS row
  static constexpr int VPR = ROWB / 16;      // 16-byte chunks per LDS row
  static constexpr int FRAGB = 8 * ES;       // bytes one lane reads per fragment
  static constexpr int PKB = 64 * FRAGB;     // bytes of one packed fragment
};

template <int DT> struct Mma;

template <> struct Mma<DT_BF16> {
  struct Frag { u32x4 v; };
  __device__ static Frag load(const char* p) { return Frag{*(const u32x4*)p}; }
  __device__ static Frag zero() { return Frag{u32x4{0u, 0u, 0u, 0u}}; }
  __device__ static void run(f32x4& acc, const Frag& a, const Frag& b) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.v),
                                                  __builtin_bit_cast(bf16x8, b.v), acc, 0, 0, 0);
  }
};

template <> struct Mma<DT_F16> {
  struct Frag { u32x4 v; };
  __device__ static Frag load(const char* p) { return Frag{*(const u32x4*)p}; }
  __device__ static Frag zero() { return Frag{u32x4{0u, 0u, 0u, 0u}}; }
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
  __device__ static Frag zero() { return Frag{u32x4{0u, 0u, 0u, 0u}, u32x4{0u, 0u, 0u, 0u}}; }
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

// ---- swizzled 32-element LDS rows ---------------------------------------------------------
//
// Chunk c (16 bytes) of row r lives at r * ROWB + ((c ^ swz(r)) * 16).  For 64-byte rows
// (2-byte types) swz mixes bits 1..3 of the row: any 8 consecutive rows then cover the
// 8 (row parity, chunk) slots of a 128-byte bank line exactly once, and any 16 rows the
// 16 slots of a 256-byte line.  For 128-byte rows (fp32) swz = (r ^ r >> 3) & 7.
template <int DT>
__device__ __forceinline__ int swz(int r) {
  if constexpr (Geo<DT>::VPR == 4) return ((r >> 1) ^ (r >> 3)) & 3;
  else return (r ^ (r >> 3)) & 7;
}

template <int DT>
__device__ __forceinline__ int sw_off(int r, int c) {
  return r * Geo<DT>::ROWB + ((c ^ swz<DT>(r)) << 4);
}

// Fragment of rows [row0, row0 + 16) of a swizzled tile (row0 a multiple of 16).
template <int DT>
__device__ __forceinline__ typename Mma<DT>::Frag frag_sw(const char* tile, int row0) {
  const int l = lane_id();
  const int r = row0 + (l & 15);
  if constexpr (Geo<DT>::VPR == 4) {
    return Mma<DT>::load(tile + sw_off<DT>(r, l >> 4));
  } else {
    typename Mma<DT>::Frag f;
    f.lo = *(const u32x4*)(tile + sw_off<DT>(r, 2 * (l >> 4)));
    f.hi = *(const u32x4*)(tile + sw_off<DT>(r, 2 * (l >> 4) + 1));
    return f;
  }
}

// Fragment of a padded (unswizzled) k-major LDS tile: rows [row0, +16), k bytes from kbyte0.
template <int DT>
__device__ __forceinline__ typename Mma<DT>::Frag frag_at(const char* tile, int pitch,
                                                          int row0, int kbyte0) {
  const int l = lane_id();
  return Mma<DT>::load(tile + (row0 + (l & 15)) * pitch + kbyte0 + (l >> 4) * Geo<DT>::FRAGB);
}

// Packed weight fragment (nb, kb) of a [n_blocks][k_blocks] fragment-order array.
template <int DT>
__device__ __forceinline__ typename Mma<DT>::Frag frag_pk(const char* pk, int nb, int kb,
                                                          int k_blocks) {
  return Mma<DT>::load(pk + ((int64_t)nb * k_blocks + kb) * Geo<DT>::PKB +
                       lane_id() * Geo<DT>::FRAGB);
}

// Fragment of a row-major source whose rows are the fragment's 16 columns and whose k
// index is contiguous: column (n0 + l % 16) is row `row(n)` (nullptr = zero), k elements
// [k0 + 8 * (l / 16), +8) valid below klim.  `fast`: rows and k0 are 16-byte aligned and
// klim is a multiple of 8.
template <int DT, class RowPtr>
__device__ __forceinline__ typename Mma<DT>::Frag frag_rows(RowPtr row, int n0, int k0,
                                                            int klim, bool fast) {
  using T = typename Elem<DT>::T;
  const int l = lane_id();
  const T* src = row(n0 + (l & 15));
  const int k = k0 + (l >> 4) * 8;
  typename Mma<DT>::Frag f = Mma<DT>::zero();
  if (!src) return f;
  if (fast) {
    if (k < klim) f = Mma<DT>::load((const char*)(src + k));
  } else {
    T tmp[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) tmp[e] = (k + e < klim) ? src[k + e] : T(0);
    __builtin_memcpy(&f, tmp, sizeof(tmp));
  }
  return f;
}

// Transposed store of one 8 x 8 block of 16-bit elements: v[r] holds source row r (8
// elements), LDS row nb * 8 + c of chunk kb receives element c of every v[r].  Odd n
// blocks write their rows in the order c ^ 1, so the two n blocks sharing an 8-lane group
// write rows of opposite parity (distinct halves of a bank line).  The parity only
// changes v_perm_b32's byte selector (halves 0/1 of each dword) and the row address, so
// the register operands stay static.
template <int DT>
__device__ __forceinline__ void store_trans8(const u32x4 (&v)[8], char* tile, int nb, int kb) {
  const int odd = nb & 1;
  constexpr uint32_t kLow = 0x05040100u, kHigh = 0x07060302u;  // low / high halves
  const uint32_t s_even = odd ? kHigh : kLow, s_odd = odd ? kLow : kHigh;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    const uint32_t sel = (c & 1) ? s_odd : s_even;
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      o[q] = __builtin_amdgcn_perm(v[2 * q + 1][c >> 1], v[2 * q][c >> 1], sel);
    *(u32x4*)(tile + sw_off<DT>(nb * 8 + (c ^ odd), kb)) = o;
  }
}

// ---- asynchronous staging: global -> LDS without registers ---------------------------------
//
// gfx950's global_load_lds_dwordx4 copies 16 bytes per lane from the lane's own global
// address to LDS at M0 (wave-uniform base) + lane * 16, and counts against vmcnt like any
// vector load.  A wave waits for its own copies with s_waitcnt vmcnt(n); a workgroup
// barrier afterwards makes every wave's copies visible.  A tile whose LDS layout is not
// lane-linear (the swizzled row tiles) is filled by permuting which global chunk each
// lane fetches instead of where it lands.
//
// The copy is issued from inline asm on purpose: the compiler then neither waits for all
// outstanding copies before every LDS read it cannot prove disjoint from them, nor at
// every barrier, and the explicit vmcnt waits below are the only synchronisation.  In
// exchange every kernel that issues copies must wait for all of them (wait_vmcnt<0>)
// before it reads the data or exits.  M0 is saved and restored around the copy because
// the compiler reserves it and does not expect asm to change it.

// 1 KiB of zeros (never written): the source of zero fill for rows or chunks outside the
// valid range, so every lane always issues its copy.  One copy per translation unit.
static __device__ __attribute__((aligned(1024))) uint32_t g_zero_kib[256] = {0};

// async_copy16_to takes the LDS byte address itself (wave-uniform), which spares the
// generic-to-LDS pointer conversion per copy.
__device__ __forceinline__ void async_copy16_to(const void* gsrc, uint32_t lds_addr) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(lds_addr);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gsrc), "s"(lds)
      : "memory");
}

__device__ __forceinline__ void async_copy16(const void* gsrc, char* lds_wave_base) {
  const uint32_t lds = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char*)lds_wave_base);
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gsrc), "s"(lds)
      : "memory");
}

// ---- LDS transpose reads (gfx950 ds_read_b64_tr_b16) -------------------------------------
//
// Within each 16-lane group, lane i supplies the address of 4 consecutive 16-bit elements
// M[i][0..3]; lane j receives M[4e + j / 4][j % 4] for e = 0..3.  So if lane i points at
// row (k0 + i / 4), columns 4 * (i % 4) .. + 3 of a row-major tile (rows = contraction
// index), lane j receives column j of rows k0 .. k0 + 3: the MFMA operand layout, read
// straight from a tile that was stored untransposed.
typedef __attribute__((ext_vector_type(4))) short i16x4;

__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  const i16x4 v =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)p);
  uint2 u;
  __builtin_memcpy(&u, &v, 8);
  return u;
}

// ---- 16 x 4 lane transposes (ds_bpermute) ------------------------------------------------
//
// The L1's address unit takes a wave's 16-byte accesses a lane quad (lanes 4 q .. 4 q + 3)
// at a time, and a quad whose four addresses lie in one 64-byte segment costs about a
// quarter of the cycles of a quad that touches four rows (rocprofv3 TA_TA_BUSY: ~16 against
// ~64 cycles per wave access on gfx950).  The MFMA operand and accumulator layouts put the
// 16 rows of a fragment on consecutive lanes -- lane 16 c + r holds row r, 16-byte chunk c
// -- so a row-major operand read, or a row-major output written, in that order makes every
// quad touch four rows.  Such accesses are issued in the quad-major order instead -- lane
// 4 r + c holds row r, chunk c, each quad one row's 64 contiguous bytes -- and the data is
// moved between the two orders across lanes with ds_bpermute (no LDS memory involved).
//
// bperm_from_quads(): the ds_bpermute byte address that gives lane l of the MFMA order the
// value of quad-order lane 4 (l % 16) + l / 16; bperm_to_quads(): lane l of the quad order
// takes MFMA-order lane 16 (l % 4) + l / 4.
__device__ __forceinline__ int bperm_from_quads(int lane) {
  return (4 * (lane & 15) + (lane >> 4)) << 2;
}
__device__ __forceinline__ int bperm_to_quads(int lane) {
  return (16 * (lane & 3) + (lane >> 2)) << 2;
}
__device__ __forceinline__ uint32_t bperm(int addr, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_ds_bpermute(addr, (int)v);
}
__device__ __forceinline__ u32x4 bperm4(int addr, const u32x4& v) {
  return u32x4{bperm(addr, v[0]), bperm(addr, v[1]), bperm(addr, v[2]), bperm(addr, v[3])};
}

// Workgroup barrier for data that reached LDS by LDS-DMA copies the caller has already
// waited for (vmcnt) and that no wave writes with ds_* stores in between: a bare
// s_barrier plus a compiler barrier.  Unlike barrier_lds, no fence is involved, so loads
// into registers that are still in flight (prefetched operands) are not waited for.
__device__ __forceinline__ void barrier_dma() {
  asm volatile("s_barrier" ::: "memory");
}

// Workgroup barrier that orders LDS accesses only: outstanding vector-memory loads (the
// asynchronous copies of later steps) stay in flight across it.
__device__ __forceinline__ void barrier_lds() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// s_waitcnt vmcnt(n), every other counter left alone (GFX9 encoding: vmcnt bits [3:0] and
// [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// s_waitcnt lgkmcnt(0) alone (vmcnt 63, expcnt 7 = no wait on those counters).
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// vmcnt(n) for a wave-uniform run-time n; n above 31 waits down to 31 outstanding, which
// is stricter than needed and therefore safe.
__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  switch (n) {
#define NSMOE_VM(i) case i: wait_vmcnt<i>(); break;
    NSMOE_VM(0) NSMOE_VM(1) NSMOE_VM(2) NSMOE_VM(3) NSMOE_VM(4) NSMOE_VM(5) NSMOE_VM(6)
    NSMOE_VM(7) NSMOE_VM(8) NSMOE_VM(9) NSMOE_VM(10) NSMOE_VM(11) NSMOE_VM(12) NSMOE_VM(13)
    NSMOE_VM(14) NSMOE_VM(15) NSMOE_VM(16) NSMOE_VM(17) NSMOE_VM(18) NSMOE_VM(19)
    NSMOE_VM(20) NSMOE_VM(21) NSMOE_VM(22) NSMOE_VM(23) NSMOE_VM(24) NSMOE_VM(25)
    NSMOE_VM(26) NSMOE_VM(27) NSMOE_VM(28) NSMOE_VM(29) NSMOE_VM(30)
#undef NSMOE_VM
    default: wait_vmcnt<31>(); break;
  }
}

// For an S-stage copy ring: loads_of(s) is the number of copies per lane that step s
// issues; waits until step s's copies have landed while steps s + 1 .. s + S - 2 stay in
// flight (the issue for s + S - 1 comes after the wait).
template <int S, class LoadsOf>
__device__ __forceinline__ void wait_step(int s, int nsteps, LoadsOf loads_of) {
  int n = 0;
#pragma unroll
  for (int u = 1; u <= S - 2; ++u)
    if (s + u < nsteps) n += loads_of(s + u);
  wait_vmcnt_dyn(n);
}

// ---- staging: global -> registers -> swizzled LDS -------------------------------------
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
        *(u32x4*)(tile + sw_off<DT>(r, c)) = v[i];
      }
    }
  }
};

// T0 is the first thread that takes part: staging several tiles on disjoint thread
// ranges spreads the work over all waves when one tile has fewer blocks than threads.
template <int DT, int NCOLS, int NT, int T0 = 0>
struct TransStage {
  using G = Geo<DT>;
  using T = typename G::T;
  static constexpr int KB = G::KC / G::VE;  // k blocks per chunk (= chunks per LDS row)
  static constexpr int NB = NCOLS / G::VE;  // n blocks per tile
  static constexpr int NBLK = KB * NB;
  static constexpr int PER = (NBLK + NT - 1) / NT;
  u32x4 v[PER][G::VE];
  __device__ __forceinline__ static int block(int i) { return (int)threadIdx.x - T0 + i * NT; }
  __device__ __forceinline__ static bool live(int blk) {
    return blk >= 0 && ((NBLK % NT == 0 && T0 == 0) || blk < NBLK);
  }

  // Source rows k in [k0, k0 + 32) (valid below klim), columns [n0, n0 + NCOLS) (valid
  // below nlim).  scale(k) multiplies the row in fp32 before it is re-rounded; rows
  // whose rowptr is null load as zero.  Block blk covers k block (blk % KB) and n block
  // (blk / KB): the KB threads of one n block write the KB chunks of the same LDS rows.
  template <class RowPtr, class Scale>
  __device__ __forceinline__ void load(RowPtr rowptr, Scale scale, int k0, int klim, int n0,
                                       int nlim, bool fast) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int blk = block(i);
      const bool on = live(blk);
      const int kb = blk % KB, nb = blk / KB;
      const int col = n0 + nb * G::VE;
#pragma unroll
      for (int r = 0; r < G::VE; ++r) {
        v[i][r] = u32x4{0u, 0u, 0u, 0u};
        const int k = k0 + kb * G::VE + r;
        if (!on || k >= klim) continue;
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
      const int blk = block(i);
      if (!live(blk)) continue;
      const int kb = blk % KB, nb = blk / KB;
      if constexpr (G::ES == 2) {
        store_trans8<DT>(v[i], tile, nb, kb);
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          u32x4 o{v[i][0][c], v[i][1][c], v[i][2][c], v[i][3][c]};
          *(u32x4*)(tile + sw_off<DT>(nb * 4 + c, kb)) = o;
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
      const int incl = wave_scan_incl(u), aincl = wave_scan_incl(a);
      const bool hit = item >= base + incl - u && item < base + incl;
      const unsigned long long m = __ballot(hit);
      if (m) {
        const int src = __ffsll((long long)m) - 1;  // wave-uniform
        const int excl = __builtin_amdgcn_readlane(incl - u, src);
        const int aexcl = __builtin_amdgcn_readlane(aincl - a, src);
        fg = g0 + src;
        floc = item - base - excl;
        faux = abase + aexcl;
        break;
      }
      base += __builtin_amdgcn_readlane(incl, 63);
      abase += __builtin_amdgcn_readlane(aincl, 63);
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

// Runs of C consecutive work items are dealt round-robin over the 8 XCDs: the j-th
// workgroup on XCD x takes item ((j / C) * 8 + x) * C + j % C. Grids sized as an upper
// bound keep their real items at the low ids, so a contiguous split per XCD (xcd_remap)
// would leave the last XCDs with only empty items; dealing runs spreads the real items
// evenly while the C items of a run (same group, shared operand rows) share one L2.
// Ids past the last whole 8*C span map to themselves, so the map is a bijection.
__device__ __forceinline__ int xcd_deal(int bid, int grid, int C) {
  const int span = 8 * C;
  if (bid >= grid / span * span) return bid;
  const int x = bid % 8, j = bid / 8;
  return (j / C * 8 + x) * C + j % C;
}

}  // namespace nsmoe
