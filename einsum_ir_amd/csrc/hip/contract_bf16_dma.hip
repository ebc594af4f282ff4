// Instantiations of the direct-to-LDS bf16 contraction kernel: 256 x 256
// tiles, 4 waves, one per (A load mode, B load mode) in {VEC_MN, VEC_K}.
#include "contract_dma.h"

namespace etir {

namespace {

template< int MA, int MB, int BK, int STAGES >
int launch_one( ContractArgs const & a, uint32_t grid, hipStream_t stream ) {
  hipLaunchKernelGGL( ( kern::contract_dma_kernel< 256, 256, BK, 2, 2, MA, MB, STAGES > ),
                      dim3( grid ), dim3( 256 ), 0, stream, a );
  return ETIR_SUCCESS;
}

// 256 x 128 tiles, two workgroups per CU (72 KB of LDS each)
int launch_bf16_dma_256x128( int32_t ma, int32_t mb, ContractArgs const & a, uint32_t grid, hipStream_t stream ) {
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN ) {
    hipLaunchKernelGGL( ( kern::contract_dma_kernel< 256, 128, 32, 2, 2, LOAD_VEC_MN, LOAD_VEC_MN, 3, 2 > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  return fail( ETIR_COMPILATION_FAILED, "no 256x128 direct-to-LDS kernel for this load-mode combination" );
}

// CUs of the current device (one persistent workgroup each)
uint32_t device_cus() {
  int l_dev = 0;
  if( hipGetDevice( &l_dev ) != hipSuccess ) return 256;
  int l_n = 0;
  if( hipDeviceGetAttribute( &l_n, hipDeviceAttributeMultiprocessorCount, l_dev ) != hipSuccess || l_n <= 0 ) {
    return 256;
  }
  return uint32_t( l_n );
}

}  // namespace

int launch_contract_bf16_dma( int32_t ma, int32_t mb, int32_t variant, ContractArgs const & a,
                              uint32_t grid, hipStream_t stream ) {
  if( variant == 2 ) return launch_bf16_dma_256x128( ma, mb, a, grid, stream );
  if( variant == 3 && ma == LOAD_VEC_MN && mb == LOAD_VEC_MN && kern::persistent_dma_eligible( a, 256, 256 ) ) {
    static thread_local int s_dev = -1;
    static thread_local uint32_t s_cus = 256;
    int l_dev = 0;
    if( hipGetDevice( &l_dev ) == hipSuccess && l_dev != s_dev ) {
      s_dev = l_dev;
      s_cus = device_cus();
    }
    uint32_t const l_g = grid < s_cus ? grid : s_cus;
    hipLaunchKernelGGL( ( kern::contract_dma_persistent_kernel< 256, 256, 32, 2, 2, 4 > ),
                        dim3( l_g ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN ) {
    if( variant == 1 || variant == 3 ) return launch_one< LOAD_VEC_MN, LOAD_VEC_MN, 32, 4 >( a, grid, stream );
    return launch_one< LOAD_VEC_MN, LOAD_VEC_MN, 64, 2 >( a, grid, stream );
  }
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_K ) return launch_one< LOAD_VEC_MN, LOAD_VEC_K, 64, 2 >( a, grid, stream );
  if( ma == LOAD_VEC_K && mb == LOAD_VEC_MN ) return launch_one< LOAD_VEC_K, LOAD_VEC_MN, 64, 2 >( a, grid, stream );
  if( ma == LOAD_VEC_K && mb == LOAD_VEC_K )  return launch_one< LOAD_VEC_K, LOAD_VEC_K, 64, 2 >( a, grid, stream );
  return fail( ETIR_COMPILATION_FAILED, "no direct-to-LDS bf16 kernel for this load-mode combination" );
}

}  // namespace etir
