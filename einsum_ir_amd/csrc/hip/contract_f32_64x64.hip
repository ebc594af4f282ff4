// Instantiations of the contraction kernel for tile f32_64x64: one per
// (A load mode, B load mode, affine K).
#include "contract_kernel.h"

namespace etir {

int launch_contract_f32_64x64( int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                   uint32_t grid, hipStream_t stream ) {
  if( ma == LOAD_SCALAR && mb == LOAD_SCALAR && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_SCALAR, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_SCALAR && mb == LOAD_VEC_MN && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_MN, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_SCALAR && mb == LOAD_VEC_K && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_K, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_SCALAR && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_SCALAR, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_MN, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_K && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_K, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_K && mb == LOAD_SCALAR && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_SCALAR, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_K && mb == LOAD_VEC_MN && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_MN, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_K && mb == LOAD_VEC_K && kaff == false ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_K, false, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_SCALAR && mb == LOAD_SCALAR && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_SCALAR, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_SCALAR && mb == LOAD_VEC_MN && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_MN, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_SCALAR && mb == LOAD_VEC_K && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_SCALAR, LOAD_VEC_K, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_SCALAR && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_SCALAR, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_MN, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_K && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_K, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_K && mb == LOAD_SCALAR && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_SCALAR, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_K && mb == LOAD_VEC_MN && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_MN, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_K && mb == LOAD_VEC_K && kaff == true ) {
    hipLaunchKernelGGL( ( kern::contract_kernel< ETIR_FP32, 64, 64, 32, 2, 2, LOAD_VEC_K, LOAD_VEC_K, true, 1 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  return fail( ETIR_COMPILATION_FAILED, "no f32_64x64 kernel for this load-mode combination" );
}

}  // namespace etir
