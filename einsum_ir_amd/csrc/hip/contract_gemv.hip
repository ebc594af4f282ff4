// Contractions with one free side of extent 1 (kernel M == 1 or N == 1):
//   out[c][m][n] = touch( sum_k A[c][m][k] * B[c][n][k] ),  M == 1 or N == 1.
//
// Such a node is a batch of matrix-vector products (einsum-tree nodes whose
// left or right tensor holds no M or N dims, e.g. the language-model series'
// "...c,cn->...n" steps).  On an MFMA tile of 64 x 64 one of the two tile
// sides is a single row, so 63/64 of every tile is padding, and each
// workgroup stages a 64 x K operand through LDS for 64 outputs.  Here one
// thread owns one output element and reduces its whole K range in registers:
// consecutive threads take consecutive indices of the long side (n when
// M == 1, m when N == 1), so the long operand's loads coalesce when it is
// unit-stride along that side, and the short operand's address is the same
// for every thread of a C index (one broadcast cache line).  The bound is the
// long operand's HBM stream.
//
// The K sum runs in ascending k with one fp32 accumulator, the order of the
// reference's scalar backend (reference src/basic/binary/
// ContractionBackendScalar.cpp:30, kernel_madd, called once per K index by
// the loop nest of ContractionBackend.cpp:296-515); the touch kernels are
// applied once per output element as in the tiled kernels' epilogue
// (ContractionBackendTpp.cpp:84-163).
#include "etir_internal.h"
#include "contract_kernel.h"

namespace etir {

namespace {

// four consecutive elements moved as one vector
template< typename T >
struct alignas( 4 * sizeof( T ) ) V4 { T v[4]; };

template< typename T >
__device__ inline float gemv_ld( T const * p, int64_t off );
template<>
__device__ inline float gemv_ld< float >( float const * p, int64_t off ) { return p[off]; }
template<>
__device__ inline float gemv_ld< uint16_t >( uint16_t const * p, int64_t off ) {
  return kern::bf16_to_f32( p[off] );
}

// The long operand and the output are each touched once per launch: their
// loads and stores are non-temporal, so they stream past the caches instead
// of evicting the short operand and each other (lm_batch's C=128 M=1
// N=65536 K=11 node, 403 MB: 73.6 us with ordinary accesses, 70.2 with
// non-temporal loads, 69.8 with non-temporal stores, 63.6 with both)
template< typename T >
__device__ inline float gemv_ld_nt( T const * p, int64_t off );
template<>
__device__ inline float gemv_ld_nt< float >( float const * p, int64_t off ) {
  return __builtin_nontemporal_load( p + off );
}
template<>
__device__ inline float gemv_ld_nt< uint16_t >( uint16_t const * p, int64_t off ) {
  return kern::bf16_to_f32( __builtin_nontemporal_load( p + off ) );
}
__device__ inline void gemv_st_nt( float * p, float v ) { __builtin_nontemporal_store( v, p ); }
__device__ inline void gemv_st_nt( uint16_t * p, uint16_t v ) { __builtin_nontemporal_store( v, p ); }

template< typename T, bool KAFF >
__global__ __launch_bounds__( 256 ) void contract_gemv_kernel( ContractArgs a ) {
  uint64_t const l_total = uint64_t( a.C ) * uint64_t( a.M ) * uint64_t( a.N );
  uint64_t const l_e = uint64_t( blockIdx.x ) * 256 + threadIdx.x;
  if( l_e >= l_total ) return;
  // element index -> (c, m, n), n fastest (m fastest when N == 1)
  int32_t l_n, l_m, l_c;
  if( l_total <= 0xffffffffull ) {
    uint32_t const l_e32 = uint32_t( l_e );
    uint32_t const l_cm = l_e32 / uint32_t( a.N );
    l_n = int32_t( l_e32 - l_cm * uint32_t( a.N ) );
    l_c = int32_t( l_cm / uint32_t( a.M ) );
    l_m = int32_t( l_cm - uint32_t( l_c ) * uint32_t( a.M ) );
  }
  else {
    uint64_t const l_cm = l_e / uint64_t( a.N );
    l_n = int32_t( l_e - l_cm * uint64_t( a.N ) );
    l_c = int32_t( l_cm / uint64_t( a.M ) );
    l_m = int32_t( l_cm - uint64_t( l_c ) * uint64_t( a.M ) );
  }

  // the touch kernels' loads first, so they are in flight with the K loop's
  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux  = ( a.aux != nullptr ) && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
  int64_t const l_off = a.tc_out[l_c] + a.tm_out[l_m] + a.tn_out[l_n];
  float l_aux = 0.0f;
  if( l_need_aux ) {
    int64_t const l_aoff = a.tc_aux[l_c] + a.tm_aux[l_m] + a.tn_aux[l_n];
    l_aux = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.aux )[l_aoff] )
                       : reinterpret_cast< float const * >( a.aux )[l_aoff];
  }
  float l_old = 0.0f;
  if( l_read_out ) {
    l_old = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.out )[l_off] )
                       : reinterpret_cast< float const * >( a.out )[l_off];
  }

  T const * l_pa = reinterpret_cast< T const * >( a.a ) + a.tc_a[l_c] + a.tm_a[l_m];
  T const * l_pb = reinterpret_cast< T const * >( a.b ) + a.tc_b[l_c] + a.tn_b[l_n];
  auto koff_a = [&]( int32_t k ) -> int64_t { return KAFF ? int64_t( k ) * a.sk_a : int64_t( a.tk_a[k] ); };
  auto koff_b = [&]( int32_t k ) -> int64_t { return KAFF ? int64_t( k ) * a.sk_b : int64_t( a.tk_b[k] ); };

  // chunks of 8 k with all 16 loads of a chunk issued before its FMAs (a
  // rolled loop would wait for every pair), added in ascending k
  float l_v = 0.0f;
  int32_t l_k = 0;
  for( ; l_k + 8 <= a.K; l_k += 8 ) {
    float l_x[8], l_y[8];
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      l_x[l_i] = gemv_ld< T >( l_pa, koff_a( l_k + l_i ) );
      l_y[l_i] = gemv_ld_nt< T >( l_pb, koff_b( l_k + l_i ) );
    }
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) l_v = fmaf( l_x[l_i], l_y[l_i], l_v );
  }
  // the last partial chunk the same way: loads of clamped (existing) k all
  // in flight together, FMAs only for the k inside K, still ascending (a
  // rolled tail loop waited for each k's loads in turn: K = 11 meant four
  // round trips instead of two)
  if( l_k < a.K ) {
    float l_x[8], l_y[8];
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      int32_t const l_kc = min( l_k + l_i, a.K - 1 );
      l_x[l_i] = gemv_ld< T >( l_pa, koff_a( l_kc ) );
      l_y[l_i] = gemv_ld_nt< T >( l_pb, koff_b( l_kc ) );
    }
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      if( l_k + l_i < a.K ) l_v = fmaf( l_x[l_i], l_y[l_i], l_v );
    }
  }

  if( l_read_out ) l_v = l_old + l_v;
  if( l_aux_first ) l_v = l_aux + l_v;
  if( a.last_touch == ETIR_KTYPE_RELU ) l_v = fmaxf( l_v, 0.0f );
  else if( a.last_touch == ETIR_KTYPE_ADD ) l_v = l_v + l_aux;
  if( a.out_bf16 ) gemv_st_nt( reinterpret_cast< uint16_t * >( a.out ) + l_off, kern::f32_to_bf16_rne( l_v ) );
  else             gemv_st_nt( reinterpret_cast< float * >( a.out ) + l_off, l_v );
}

// Kernel M == 1 with the long operand B and the output unit-stride along N
// (a.gemv_v4): each thread takes 4 consecutive n, one 4-element vector of B
// per k (16 bytes fp32, 8 bytes bf16) and one vector store, each output
// summed in ascending k with its own accumulator exactly as above.  The
// short operand A is one value per k for all four.  Aux values are read per
// element (the aux tensor may broadcast along n).
template< typename T, bool KAFF >
__global__ __launch_bounds__( 256 ) void contract_gemv4_kernel( ContractArgs a ) {
  typedef float f4 __attribute__( ( ext_vector_type( 4 ) ) );
  int32_t const l_n4 = a.N / 4;
  uint64_t const l_total = uint64_t( a.C ) * uint64_t( l_n4 );
  uint64_t const l_e = uint64_t( blockIdx.x ) * 256 + threadIdx.x;
  if( l_e >= l_total ) return;
  int32_t l_c, l_q;
  if( l_total <= 0xffffffffull ) {
    l_c = int32_t( uint32_t( l_e ) / uint32_t( l_n4 ) );
    l_q = int32_t( uint32_t( l_e ) - uint32_t( l_c ) * uint32_t( l_n4 ) );
  }
  else {
    l_c = int32_t( l_e / uint64_t( l_n4 ) );
    l_q = int32_t( l_e - uint64_t( l_c ) * uint64_t( l_n4 ) );
  }
  int32_t const l_n = 4 * l_q;

  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux  = ( a.aux != nullptr ) && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
  int64_t const l_off = a.tc_out[l_c] + a.tm_out[0] + l_n;
  float l_aux[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
  if( l_need_aux ) {
    int64_t const l_ab = a.tc_aux[l_c] + a.tm_aux[0];
#pragma unroll
    for( int l_i = 0; l_i < 4; l_i++ ) {
      int64_t const l_aoff = l_ab + a.tn_aux[l_n + l_i];
      l_aux[l_i] = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.aux )[l_aoff] )
                              : reinterpret_cast< float const * >( a.aux )[l_aoff];
    }
  }
  float l_old[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
  if( l_read_out ) {
    if( a.out_bf16 ) {
      V4< uint16_t > const l_o = *reinterpret_cast< V4< uint16_t > const * >(
          reinterpret_cast< uint16_t const * >( a.out ) + l_off );
#pragma unroll
      for( int l_i = 0; l_i < 4; l_i++ ) l_old[l_i] = kern::bf16_to_f32( l_o.v[l_i] );
    }
    else {
      f4 const l_o = *reinterpret_cast< f4 const * >( reinterpret_cast< float const * >( a.out ) + l_off );
#pragma unroll
      for( int l_i = 0; l_i < 4; l_i++ ) l_old[l_i] = l_o[l_i];
    }
  }

  T const * l_pa = reinterpret_cast< T const * >( a.a ) + a.tc_a[l_c] + a.tm_a[0];
  T const * l_pb = reinterpret_cast< T const * >( a.b ) + a.tc_b[l_c] + l_n;
  auto koff_a = [&]( int32_t k ) -> int64_t { return KAFF ? int64_t( k ) * a.sk_a : int64_t( a.tk_a[k] ); };
  auto koff_b = [&]( int32_t k ) -> int64_t { return KAFF ? int64_t( k ) * a.sk_b : int64_t( a.tk_b[k] ); };
  // one non-temporal vector of 4 elements of B (16 bytes fp32, 8 bytes bf16)
  typedef uint16_t u16x4 __attribute__( ( ext_vector_type( 4 ) ) );
  auto ld4 = [&]( int64_t off ) {
    f4 l_r;
    if constexpr( sizeof( T ) == 4 ) {
      l_r = __builtin_nontemporal_load( reinterpret_cast< f4 const * >( l_pb + off ) );
    }
    else {
      u16x4 const l_t = __builtin_nontemporal_load( reinterpret_cast< u16x4 const * >( l_pb + off ) );
#pragma unroll
      for( int l_i = 0; l_i < 4; l_i++ ) l_r[l_i] = kern::bf16_to_f32( l_t[l_i] );
    }
    return l_r;
  };

  float l_v[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
  int32_t l_k = 0;
  for( ; l_k + 8 <= a.K; l_k += 8 ) {
    float l_x[8];
    f4    l_y[8];
#pragma unroll
    for( int l_j = 0; l_j < 8; l_j++ ) {
      l_x[l_j] = gemv_ld< T >( l_pa, koff_a( l_k + l_j ) );
      l_y[l_j] = ld4( koff_b( l_k + l_j ) );
    }
#pragma unroll
    for( int l_j = 0; l_j < 8; l_j++ )
#pragma unroll
      for( int l_i = 0; l_i < 4; l_i++ ) l_v[l_i] = fmaf( l_x[l_j], l_y[l_j][l_i], l_v[l_i] );
  }
  if( l_k < a.K ) {
    // the last partial chunk: clamped loads in flight together, as above
    float l_x[8];
    f4    l_y[8];
#pragma unroll
    for( int l_j = 0; l_j < 8; l_j++ ) {
      int32_t const l_kc = min( l_k + l_j, a.K - 1 );
      l_x[l_j] = gemv_ld< T >( l_pa, koff_a( l_kc ) );
      l_y[l_j] = ld4( koff_b( l_kc ) );
    }
#pragma unroll
    for( int l_j = 0; l_j < 8; l_j++ ) {
      if( l_k + l_j < a.K ) {
#pragma unroll
        for( int l_i = 0; l_i < 4; l_i++ ) l_v[l_i] = fmaf( l_x[l_j], l_y[l_j][l_i], l_v[l_i] );
      }
    }
  }

  float l_r[4];
#pragma unroll
  for( int l_i = 0; l_i < 4; l_i++ ) {
    float l_w = l_v[l_i];
    if( l_read_out ) l_w = l_old[l_i] + l_w;
    if( l_aux_first ) l_w = l_aux[l_i] + l_w;
    if( a.last_touch == ETIR_KTYPE_RELU ) l_w = fmaxf( l_w, 0.0f );
    else if( a.last_touch == ETIR_KTYPE_ADD ) l_w = l_w + l_aux[l_i];
    l_r[l_i] = l_w;
  }
  if( a.out_bf16 ) {
    u16x4 l_o;
#pragma unroll
    for( int l_i = 0; l_i < 4; l_i++ ) l_o[l_i] = kern::f32_to_bf16_rne( l_r[l_i] );
    __builtin_nontemporal_store( l_o, reinterpret_cast< u16x4 * >( reinterpret_cast< uint16_t * >( a.out ) + l_off ) );
  }
  else {
    __builtin_nontemporal_store( f4{ l_r[0], l_r[1], l_r[2], l_r[3] },
                                 reinterpret_cast< f4 * >( reinterpret_cast< float * >( a.out ) + l_off ) );
  }
}

}  // namespace

int launch_contract_gemv( bool bf16_in, ContractArgs const & a, hipStream_t stream ) {
  int64_t const l_total = int64_t( a.C ) * a.M * a.N;
  if( l_total == 0 ) return ETIR_SUCCESS;
  int64_t const l_esz = bf16_in ? 2 : 4;
  // vector accesses need the long operand's and the output's base addresses
  // aligned to one vector
  bool const l_v4 = a.gemv_v4 && a.M == 1 && reinterpret_cast< uintptr_t >( a.b ) % uintptr_t( 4 * l_esz ) == 0
                 && reinterpret_cast< uintptr_t >( a.out ) % uintptr_t( a.out_bf16 ? 8 : 16 ) == 0;
  int64_t const l_blocks = ( ( l_v4 ? l_total / 4 : l_total ) + 255 ) / 256;
  if( l_blocks > 0x7fffffffLL ) return fail( ETIR_UNDEFINED_ERROR, "gemv contraction: grid too large" );
  dim3 const l_grid( (uint32_t) l_blocks );
  bool const l_kaff = ( a.k_affine != 0 );
  auto go = [&]( auto t_c, auto kaff_c ) {
    typedef typename decltype( t_c )::type T;
    constexpr bool KA = decltype( kaff_c )::value;
    if( l_v4 ) hipLaunchKernelGGL( ( contract_gemv4_kernel< T, KA > ), l_grid, dim3( 256 ), 0, stream, a );
    else       hipLaunchKernelGGL( ( contract_gemv_kernel< T, KA > ), l_grid, dim3( 256 ), 0, stream, a );
  };
  struct F32 { typedef float type; };
  struct BF16 { typedef uint16_t type; };
  if( bf16_in ) {
    if( l_kaff ) go( BF16(), std::true_type() );
    else         go( BF16(), std::false_type() );
  }
  else {
    if( l_kaff ) go( F32(), std::true_type() );
    else         go( F32(), std::false_type() );
  }
  return ETIR_SUCCESS;
}

}  // namespace etir
