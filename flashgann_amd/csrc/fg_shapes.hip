// fg_shapes.hip -- one shape class of the search kernel per object file:
// compiled once for each FG_SHAPE = 0 .. 6 (see the Makefile), so the
// classes' kernels compile in parallel.  fg_search.hip's launch_t picks the
// class (fg_kernel.hpp declares the seven launch functions).
#include "fg_kernel.hpp"

#ifndef FG_SHAPE
#error "compile with -DFG_SHAPE=0..6"
#endif

namespace fgk {

#define FG_SHAPE_ARGS                                                                                  \
    const SearchParams &P, hipStream_t stream, bool count, bool prof, int *waves_only, bool one_wave, \
        long long *resident
#define FG_SHAPE_CALL P, stream, count, prof, waves_only, one_wave, resident

#if FG_SHAPE == 0
void launch_shape0(FG_SHAPE_ARGS) { launch_geo<4, 4, 128, 32>(FG_SHAPE_CALL); }  // d 128 / degree 32
#elif FG_SHAPE == 1
void launch_shape1(FG_SHAPE_ARGS) { launch_geo<4, 3, 96, 32>(FG_SHAPE_CALL); }  // d 96 / degree 32
#elif FG_SHAPE == 2
void launch_shape2(FG_SHAPE_ARGS) { launch_geo<4, 3, 96, 16>(FG_SHAPE_CALL); }  // d 96 / degree 16
#elif FG_SHAPE == 3
void launch_shape3(FG_SHAPE_ARGS) { launch_geo<2, 2, 0, 0>(FG_SHAPE_CALL); }  // padded dim 64
#elif FG_SHAPE == 4
void launch_shape4(FG_SHAPE_ARGS) { launch_geo<4, 3, 0, 0>(FG_SHAPE_CALL); }  // padded 128, d <= 96
#elif FG_SHAPE == 5
void launch_shape5(FG_SHAPE_ARGS) { launch_geo<4, 4, 0, 0>(FG_SHAPE_CALL); }  // padded 128
#elif FG_SHAPE == 6
void launch_shape6(FG_SHAPE_ARGS) { launch_geo<0, 0, 0, 0>(FG_SHAPE_CALL); }  // padded dim >= 256
#else
#error "FG_SHAPE must be 0..6"
#endif

}  // namespace fgk
