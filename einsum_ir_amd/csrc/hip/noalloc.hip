// Allocation-free contraction entry point (etir_hip_contraction_execute_noalloc)
// and the offset-table fill kernel it plans with.
//
// etir_hip_contraction_create allocates device memory for a plan's offset
// tables and, for split-K plans, its workspace.  Callers that cannot
// allocate (code under stream capture, tight serving loops, harnesses that
// forbid hipMalloc) instead plan and execute in one call whose device memory
// is carved from `scratch`, a file-scope array of kScratchBytes that every
// GPU the library runs on holds until the process ends.  The tables are
// generated into it by fill_tables_kernel from the loop sizes and strides
// (kernel arguments only: no allocation, no host-to-device copy); the split-K
// partial sums go after them.  Every call on one GPU shares that GPU's array:
// calls that overlap on one GPU (different streams, or different host
// threads) race.  Nothing in the array needs clearing between calls: the
// tables are written whole before use and every workspace slice is written
// whole by the partial contraction before the reduction reads it.
#include "etir_internal.h"
#include <array>
#include <mutex>

namespace etir {

// 64 MiB: tables of any BASELINE contraction (~0.1 MB) plus the split-K
// workspace of contractions with outputs up to ~4M floats at S = 4
constexpr std::size_t kScratchBytes = std::size_t( 64 ) << 20;

static __device__ __align__( 256 ) char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
std::array< char *, kMaxDevices > g_scratch_ptr{};   // device address of `scratch`, per device

// device address of this device's copy of `scratch` (looked up once per
// device, with that device current)
int scratch_of_current_device( char ** o_ptr ) {
  int l_dev = 0;
  ETIR_HIP_CHECK( hipGetDevice( &l_dev ) );
  if( l_dev < 0 || l_dev >= kMaxDevices ) return fail( ETIR_UNDEFINED_ERROR, "device index out of range" );
  std::lock_guard< std::mutex > l_lock( g_scratch_mutex );
  if( g_scratch_ptr[l_dev] == nullptr ) {
    void * l_p = nullptr;
    hipError_t const l_e = hipGetSymbolAddress( &l_p, HIP_SYMBOL( scratch ) );
    if( l_e != hipSuccess || l_p == nullptr ) {
      return fail( ETIR_UNDEFINED_ERROR, std::string( "hipGetSymbolAddress(scratch) failed: " )
                                         + hipGetErrorString( l_e ) );
    }
    g_scratch_ptr[l_dev] = static_cast< char * >( l_p );
  }
  *o_ptr = g_scratch_ptr[l_dev];
  return ETIR_SUCCESS;
}

__global__ __launch_bounds__( 256 )
void fill_tables_kernel( TableFill f, char * base ) {
  for( int64_t l_e = int64_t( blockIdx.x ) * blockDim.x + threadIdx.x; l_e < f.count;
       l_e += int64_t( gridDim.x ) * blockDim.x ) {
    int64_t l_off[4] = { 0, 0, 0, 0 };
    int64_t l_idx = l_e;
    for( int l_d = f.ndims - 1; l_d >= 0; l_d-- ) {
      int64_t const l_digit = l_idx % f.sizes[l_d];
      l_idx /= f.sizes[l_d];
      for( int l_t = 0; l_t < f.ntab; l_t++ ) l_off[l_t] += l_digit * f.strides[l_t][l_d];
    }
    for( int l_t = 0; l_t < f.ntab; l_t++ ) {
      if( f.is64 ) reinterpret_cast< int64_t * >( base + f.dst[l_t] )[l_e] = l_off[l_t];
      else         reinterpret_cast< int32_t * >( base + f.dst[l_t] )[l_e] = int32_t( l_off[l_t] );
    }
  }
}

}  // namespace

int launch_fill_tables( TableFill const & f, char * base, hipStream_t stream ) {
  if( f.ndims < 0 || f.ndims > kFillMaxDims || f.ntab < 1 || f.ntab > 4 ) {
    return fail( ETIR_UNDEFINED_ERROR, "fill_tables: bad descriptor" );
  }
  for( int l_d = 0; l_d < f.ndims; l_d++ ) {
    if( f.sizes[l_d] <= 0 ) return fail( ETIR_UNDEFINED_ERROR, "fill_tables: non-positive loop size" );
  }
  int64_t const l_blocks = std::min< int64_t >( ( f.count + 255 ) / 256, 1024 );
  hipLaunchKernelGGL( fill_tables_kernel, dim3( (uint32_t) l_blocks ), dim3( 256 ), 0, stream, f, base );
  hipError_t const l_e = hipGetLastError();
  if( l_e != hipSuccess ) {
    return fail( ETIR_UNDEFINED_ERROR, std::string( "fill_tables launch failed: " ) + hipGetErrorString( l_e ) );
  }
  return ETIR_SUCCESS;
}

}  // namespace etir

extern "C" int etir_hip_contraction_execute_noalloc( int64_t         num_loops,
                                                     int32_t const * dim_types,
                                                     int64_t const * sizes,
                                                     int64_t const * strides_left,
                                                     int64_t const * strides_right,
                                                     int64_t const * strides_out_aux,
                                                     int64_t const * strides_out,
                                                     int32_t         dtype_left,
                                                     int32_t         dtype_right,
                                                     int32_t         dtype_comp,
                                                     int32_t         dtype_out,
                                                     int32_t         ktype_first_touch,
                                                     int32_t         ktype_main,
                                                     int32_t         ktype_last_touch,
                                                     void const    * left,
                                                     void const    * right,
                                                     void const    * out_aux,
                                                     void          * out,
                                                     void          * stream ) {
  char * l_scratch = nullptr;
  int l_err = etir::scratch_of_current_device( &l_scratch );
  if( l_err != ETIR_SUCCESS ) return l_err;
  etir::DevicePlacement l_place;
  l_place.base = l_scratch;
  l_place.capacity = etir::kScratchBytes;
  l_place.stream = reinterpret_cast< hipStream_t >( stream );
  etir::ContractionPlan l_plan;
  l_err = etir::plan_contraction( num_loops, dim_types, sizes, strides_left, strides_right, strides_out_aux,
                                  strides_out, dtype_left, dtype_right, dtype_comp, dtype_out,
                                  ktype_first_touch, ktype_main, ktype_last_touch, l_plan, &l_place );
  if( l_err == ETIR_SUCCESS ) {
    l_err = etir::launch_contraction( l_plan, left, right, out_aux, out, l_place.stream );
  }
  etir::release_contraction( l_plan );   // placed: frees nothing
  return l_err;
}
