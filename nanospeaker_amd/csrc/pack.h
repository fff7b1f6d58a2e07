// Geometry of the fragment-order weight packs (pack.hip) shared with the expert kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace nsmoe {

struct PackGeom {
  int hp;         // gate (and up) column span of the packed W_in: 64, 128 or 256
  int in_kb;      // k blocks (32) of packed W_in: ceil(d / 32)
  int in_nb;      // column blocks (16) of packed W_in: 2 * hp / 16
  int out_kb;     // k blocks of packed W_out: ceil(H / 32)
  int out_nb;     // column blocks of packed W_out: ceil(d / 64) * 4
  size_t in_bytes, out_bytes;  // whole stacks (routed + shared groups)
};

PackGeom pack_geom(int dtype, int d, int H, int E, int S);

int pack_weights(int dtype, const void* w_in, const void* w_out, const void* w_sh_in,
                 const void* w_sh_out, int E, int S, int d, int H, void* p_in, void* p_out,
                 hipStream_t s);

}  // namespace nsmoe
