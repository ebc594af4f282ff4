// Explicit instantiations of the f32 contraction kernels and their dispatch.
// One explicit instantiation per (tile, A load mode, B load mode).
#include "contract_kernel.h"

namespace etir {

int launch_contract_f32( int32_t tile, int32_t ma, int32_t mb, ContractArgs const & a,
                         uint32_t grid, hipStream_t stream ) {
  if( tile == TILE_F32_128x128 ) {
    if( ma == LOAD_SCALAR && mb == LOAD_SCALAR ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_SCALAR, LOAD_SCALAR > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_SCALAR && mb == LOAD_VEC_MN ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_MN > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_SCALAR && mb == LOAD_VEC_K ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_K > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_MN && mb == LOAD_SCALAR ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_VEC_MN, LOAD_SCALAR > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_MN > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_MN && mb == LOAD_VEC_K ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_K > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_K && mb == LOAD_SCALAR ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_VEC_K, LOAD_SCALAR > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_K && mb == LOAD_VEC_MN ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_MN > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_K && mb == LOAD_VEC_K ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 128, 128, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_K > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
  }
  if( tile == TILE_F32_64x64 ) {
    if( ma == LOAD_SCALAR && mb == LOAD_SCALAR ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_SCALAR > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_SCALAR && mb == LOAD_VEC_MN ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_MN > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_SCALAR && mb == LOAD_VEC_K ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_K > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_MN && mb == LOAD_SCALAR ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_SCALAR > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_MN > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_MN && mb == LOAD_VEC_K ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_K > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_K && mb == LOAD_SCALAR ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_SCALAR > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_K && mb == LOAD_VEC_MN ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_MN > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
    if( ma == LOAD_VEC_K && mb == LOAD_VEC_K ) {
      hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_K > ),
                          dim3( grid ), dim3( 256 ), 0, stream, a );
      return ETIR_SUCCESS;
    }
  }
  return fail( ETIR_COMPILATION_FAILED, "no f32 contraction kernel for this tile/load-mode combination" );
}

}  // namespace etir
