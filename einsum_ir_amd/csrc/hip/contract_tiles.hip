// The generic contraction kernel of contract_kernel.h at its six tile shapes,
// behind one dispatcher.  Each tile is instantiated for every pair of operand
// load modes (nine for bf16; 25 for fp32, whose tiles also take the 8-byte
// vector modes), with and without an affine K offset; a workgroup has one
// wave per (M, N) wave position.
//
//   tile                 dtype  BM   BN   BK  waves (M x N)  min waves per SIMD (launch bound)
//   TILE_F32_128x128     fp32   128  128  32  4 x 2          1
//   TILE_F32_64x64       fp32    64   64  32  2 x 2          1
//   TILE_BF16_256x256    bf16   256  256  64  2 x 4          2
//   TILE_BF16_256x128    bf16   256  128  32  2 x 2          2
//   TILE_BF16_128x128    bf16   128  128  64  2 x 2          1
//   TILE_BF16_64x64      bf16    64   64  64  2 x 2          1
//
// fp32 128 x 128 runs 8 waves of 32 x 64: with two workgroups per CU (LDS)
// that is four waves per SIMD, against two for 4 waves of 64 x 64 (same
// speed where each CU has several tiles, 6-8 % faster where it has one).
#include "contract_kernel.h"

namespace etir {

namespace {

template< int DT, int BM, int BN, int BK, int WM, int WN, int WPE >
int launch_tile( int32_t ma, int32_t mb, bool kaff, ContractArgs const & a, uint32_t grid,
                 hipStream_t stream ) {
  return with_load_modes< DT == ETIR_FP32 >( ma, mb, kaff, [&]( auto i_ma, auto i_mb, auto i_kaff ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< DT, BM, BN, BK, WM, WN, decltype( i_ma )::value,
                                                 decltype( i_mb )::value, decltype( i_kaff )::value, WPE > ),
                        dim3( grid ), dim3( 64 * WM * WN ), 0, stream, a );
    return int( ETIR_SUCCESS );
  } );
}

}  // namespace

int launch_contract_tile( int32_t tile, int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                          uint32_t grid, hipStream_t stream ) {
  switch( tile ) {
    case TILE_F32_128x128:  return launch_tile< ETIR_FP32, 128, 128, 32, 4, 2, 1 >( ma, mb, kaff, a, grid, stream );
    case TILE_F32_64x64:    return launch_tile< ETIR_FP32,  64,  64, 32, 2, 2, 1 >( ma, mb, kaff, a, grid, stream );
    case TILE_BF16_256x256: return launch_tile< ETIR_BF16, 256, 256, 64, 2, 4, 2 >( ma, mb, kaff, a, grid, stream );
    case TILE_BF16_256x128: return launch_tile< ETIR_BF16, 256, 128, 32, 2, 2, 2 >( ma, mb, kaff, a, grid, stream );
    case TILE_BF16_128x128: return launch_tile< ETIR_BF16, 128, 128, 64, 2, 2, 1 >( ma, mb, kaff, a, grid, stream );
    case TILE_BF16_64x64:   return launch_tile< ETIR_BF16,  64,  64, 64, 2, 2, 1 >( ma, mb, kaff, a, grid, stream );
    default: return fail( ETIR_COMPILATION_FAILED, "contraction: no generic kernel for this tile" );
  }
}

}  // namespace etir
