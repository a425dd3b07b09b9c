// Every GEMM kernel of libsys1hip in one translation unit: the tile and
// skinny shapes of shapes.def, expanded here instead of one file per shape.
// For builds that want a fixed list of sources (a Rust build.rs, a Makefile):
//   hipcc --offload-arch=gfx950 ... -shared sys1hip.hip chain.hip shapes_all.hip
// links the same library as sys1_amd/build.py, which compiles the shapes in
// parallel, one per translation unit, from the same list.
#include "gemm_tile.hpp"
#include "skinny.hpp"
#include "kernel_fns.hpp"

#define SYS1_SHAPE(name, BM, BN, WM, WN, ST, BK, OCC, SK, PW, EFF, SWEFF, LKEFF) \
  SYS1_DEFINE_SHAPE(name, BM, BN, WM, WN, ST, BK, OCC, SK, PW)
#define SYS1_SKINNY(name, FM, FN, NW, U) SYS1_DEFINE_SKINNY(name, FM, FN, NW, U)
#include "shapes.def"
#undef SYS1_SHAPE
#undef SYS1_SKINNY
