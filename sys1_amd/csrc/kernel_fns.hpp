// The kernel-function table of one GEMM tile shape: every epilogue's
// instantiation of gemm_tile_kernel.  A shape's table is defined in a
// translation unit of its own (SYS1_DEFINE_SHAPE) and declared wherever the
// dispatcher needs it (SYS1_DECLARE_SHAPE), so the shapes compile in
// parallel.
#pragma once

#include "common.hpp"

namespace sys1 {

using KernelFn = void (*)(GemmArgs);

}  // namespace sys1

#define SYS1_DECLARE_SHAPE(name) \
  namespace sys1 {               \
  extern const KernelFn name##_fns[kEpiCount]; \
  }

#ifdef SYS1_GEMM_TILE_HPP
namespace sys1 {
// The conv epilogues exist for shapes whose waves hold every row of a tile.
template <int BM, int BN, int WM, int WN, int ST, int BK, int OCC, bool SK, int EPI, int PW>
constexpr KernelFn conv_fn() {
  if constexpr (WM == 1 && PW == 0) return gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, EPI, PW>;
  else return nullptr;
}
}  // namespace sys1

#define SYS1_DEFINE_SHAPE(name, BM, BN, WM, WN, ST, BK, OCC, SK, PW)                              \
  namespace sys1 {                                                                                \
  extern const KernelFn name##_fns[kEpiCount];                                                    \
  const KernelFn name##_fns[kEpiCount] = {                                                        \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 0, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 1, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 2, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 3, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 4, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 5, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 6, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 7, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 8, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 9, PW>,                                   \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 10, PW>,                                  \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 11, PW>,                                  \
      conv_fn<BM, BN, WM, WN, ST, BK, OCC, SK, 12, PW>(),                                         \
      conv_fn<BM, BN, WM, WN, ST, BK, OCC, SK, 13, PW>(),                                         \
      gemm_tile_kernel<BM, BN, WM, WN, ST, BK, OCC, SK, 14, PW>};                                 \
  }
#endif

#ifdef SYS1_SKINNY_HPP
namespace sys1 {
// A skinny-M kernel per epilogue; null where the epilogue does not apply
// (gated epilogues need whole 32-row gate/up groups, an even FN; RoPE and
// conv run on the tile kernels).
template <int FM, int FN, int NW, int U, int EPI>
constexpr KernelFn skinny_fn() {
  if constexpr ((epi_gated(EPI) && FN % 2 != 0) || epi_base(EPI) == kEpiRopeQkv || epi_base(EPI) == kEpiConvSilu)
    return nullptr;
  else
    return skinny_kernel<FM, FN, NW, U, EPI>;
}
}  // namespace sys1

#define SYS1_DEFINE_SKINNY(name, FM, FN, NW, U)                                                              \
  namespace sys1 {                                                                                          \
  extern const KernelFn name##_fns[kEpiCount];                                                              \
  const KernelFn name##_fns[kEpiCount] = {                                                                  \
      skinny_fn<FM, FN, NW, U, 0>(),  skinny_fn<FM, FN, NW, U, 1>(),  skinny_fn<FM, FN, NW, U, 2>(),        \
      skinny_fn<FM, FN, NW, U, 3>(),  skinny_fn<FM, FN, NW, U, 4>(),  skinny_fn<FM, FN, NW, U, 5>(),        \
      skinny_fn<FM, FN, NW, U, 6>(),  skinny_fn<FM, FN, NW, U, 7>(),  skinny_fn<FM, FN, NW, U, 8>(),        \
      skinny_fn<FM, FN, NW, U, 9>(),  skinny_fn<FM, FN, NW, U, 10>(), skinny_fn<FM, FN, NW, U, 11>(),       \
      skinny_fn<FM, FN, NW, U, 12>(), skinny_fn<FM, FN, NW, U, 13>(), skinny_fn<FM, FN, NW, U, 14>()};      \
  }
#endif
