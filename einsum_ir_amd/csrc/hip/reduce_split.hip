// Second half of a split-K contraction: out = touch( sum_s ws[s] ).
//
// The partial contraction wrote slice s of the workspace at the output's own
// offsets (tc_out[c] + tm_out[m] + tn_out[n]) plus s * span; this kernel sums
// the S slices in ascending s (a fixed order, so results are reproducible)
// and applies the first/last-touch kernels of the reference's loop nest once
// per output element (reference src/basic/binary/ContractionBackendTpp.cpp:
// 84-163: ZERO/COPY/ADD first touch, RELU/ADD last touch, aux broadcasts via
// zero strides).  One thread per output element; consecutive threads take
// consecutive kernel-N indices, the output's unit-stride index when it has one.
// A dense output takes the flat kernel below instead (with an aux tensor,
// where that broadcasts over the output's outermost loops only).
#include "etir_internal.h"
#include "contract_kernel.h"

namespace etir {

namespace {

__global__ __launch_bounds__( 256 ) void split_reduce_kernel( SplitReduceArgs a ) {
  // element index -> (c, m, n); 32-bit division when the index range allows
  // (the common case: 64-bit division is a long instruction sequence)
  uint64_t const l_total = uint64_t( a.C ) * uint64_t( a.M ) * uint64_t( a.N );
  uint64_t const l_e = uint64_t( blockIdx.x ) * 256 + threadIdx.x;
  if( l_e >= l_total ) return;
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
  int64_t const l_off = a.tc_out[l_c] + a.tm_out[l_m] + a.tn_out[l_n];

  // the touch kernels' loads (old output, aux) are issued first, then the
  // slices in chunks of 8 with every load of a chunk in flight together (a
  // rolled loop would wait for each slice before loading the next); the
  // slices are added in ascending order, a fixed order
  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux  = ( a.aux != nullptr ) && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
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

  float l_v = 0.0f;
  float const * l_p = a.ws + l_off;
  for( int32_t l_s = 0; l_s < a.S; l_s += 8 ) {
    float l_x[8];
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      l_x[l_i] = ( l_s + l_i < a.S ) ? l_p[int64_t( l_s + l_i ) * a.span] : 0.0f;
    }
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      if( l_s + l_i < a.S ) l_v += l_x[l_i];
    }
  }
  if( l_read_out ) l_v = l_old + l_v;
  if( l_aux_first ) l_v = l_aux + l_v;
  if( a.last_touch == ETIR_KTYPE_RELU ) l_v = fmaxf( l_v, 0.0f );
  else if( a.last_touch == ETIR_KTYPE_ADD ) l_v = l_v + l_aux;
  if( a.out_bf16 ) reinterpret_cast< uint16_t * >( a.out )[l_off] = kern::f32_to_bf16_rne( l_v );
  else             reinterpret_cast< float * >( a.out )[l_off] = l_v;
}

// A dense output (its offsets exactly 0 .. n_flat - 1): the slices and the
// output as flat arrays, VEC consecutive elements per thread (16-byte loads
// of fp32 slices), no offset tables and no index division; an aux tensor
// that broadcasts over the output's outermost loops is read at o % flat_aux.
// Same ascending slice order and touch kernels as above, per element.
template< int VEC >
__global__ __launch_bounds__( 256 ) void split_reduce_flat_kernel( SplitReduceArgs a ) {
  typedef float FV __attribute__( ( ext_vector_type( VEC ) ) );
  int64_t const l_o = ( int64_t( blockIdx.x ) * 256 + threadIdx.x ) * VEC;
  if( l_o >= a.n_flat ) return;
  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux  = ( a.aux != nullptr ) && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
  // the last thread may hold fewer than VEC elements: element by element
  int const l_n = int( min( int64_t( VEC ), a.n_flat - l_o ) );
  FV l_aux = FV( 0.0f );
  if( l_need_aux ) {
    // one 64-bit division per thread: the next elements' aux offsets wrap at
    // most once per element
    int64_t l_ao = l_o % a.flat_aux;
#pragma unroll
    for( int l_j = 0; l_j < VEC; l_j++ ) {
      if( l_j > 0 && ++l_ao == a.flat_aux ) l_ao = 0;
      if( l_j < l_n ) {
        l_aux[l_j] = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.aux )[l_ao] )
                                : reinterpret_cast< float const * >( a.aux )[l_ao];
      }
    }
  }
  FV l_old = FV( 0.0f );
  if( l_read_out ) {
#pragma unroll
    for( int l_j = 0; l_j < VEC; l_j++ ) {
      if( l_j < l_n ) {
        l_old[l_j] = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.out )[l_o + l_j] )
                                : reinterpret_cast< float const * >( a.out )[l_o + l_j];
      }
    }
  }
  FV l_v = FV( 0.0f );
  float const * l_p = a.ws + l_o;
  for( int32_t l_s = 0; l_s < a.S; l_s += 8 ) {
    FV l_x[8];
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      l_x[l_i] = FV( 0.0f );
      if( l_s + l_i < a.S ) {
        float const * l_q = l_p + int64_t( l_s + l_i ) * a.span;
        if( VEC > 1 && l_n == VEC ) l_x[l_i] = *reinterpret_cast< FV const * >( l_q );
        else {
#pragma unroll
          for( int l_j = 0; l_j < VEC; l_j++ ) if( l_j < l_n ) l_x[l_i][l_j] = l_q[l_j];
        }
      }
    }
#pragma unroll
    for( int l_i = 0; l_i < 8; l_i++ ) {
      if( l_s + l_i < a.S ) l_v += l_x[l_i];
    }
  }
#pragma unroll
  for( int l_j = 0; l_j < VEC; l_j++ ) {
    float l_e = l_v[l_j];
    if( l_read_out ) l_e = l_old[l_j] + l_e;
    if( l_aux_first ) l_e = l_aux[l_j] + l_e;
    if( a.last_touch == ETIR_KTYPE_RELU ) l_e = fmaxf( l_e, 0.0f );
    else if( a.last_touch == ETIR_KTYPE_ADD ) l_e = l_e + l_aux[l_j];
    l_v[l_j] = l_e;
  }
  if( a.out_bf16 ) {
    uint16_t * l_out = reinterpret_cast< uint16_t * >( a.out ) + l_o;
#pragma unroll
    for( int l_j = 0; l_j < VEC; l_j++ ) if( l_j < l_n ) l_out[l_j] = kern::f32_to_bf16_rne( l_v[l_j] );
  }
  else {
    float * l_out = reinterpret_cast< float * >( a.out ) + l_o;
    if( VEC > 1 && l_n == VEC ) *reinterpret_cast< FV * >( l_out ) = l_v;
    else {
#pragma unroll
      for( int l_j = 0; l_j < VEC; l_j++ ) if( l_j < l_n ) l_out[l_j] = l_v[l_j];
    }
  }
}

}  // namespace

int launch_split_reduce( SplitReduceArgs const & a, hipStream_t stream ) {
  if( a.n_flat > 0 ) {
    if( a.aux != nullptr && a.flat_aux <= 0 ) {
      return fail( ETIR_UNDEFINED_ERROR, "split reduce: flat reduction with an aux tensor but no aux period" );
    }
    int64_t const l_vec = a.flat_vec ? 4 : 1;
    int64_t const l_blocks = ( a.n_flat + 256 * l_vec - 1 ) / ( 256 * l_vec );
    if( l_blocks > 0x7fffffffLL ) return fail( ETIR_UNDEFINED_ERROR, "split reduce: grid too large" );
    if( a.flat_vec ) hipLaunchKernelGGL( split_reduce_flat_kernel< 4 >, dim3( (uint32_t) l_blocks ), dim3( 256 ), 0, stream, a );
    else             hipLaunchKernelGGL( split_reduce_flat_kernel< 1 >, dim3( (uint32_t) l_blocks ), dim3( 256 ), 0, stream, a );
    return ETIR_SUCCESS;
  }
  int64_t const l_total = int64_t( a.C ) * a.M * a.N;
  if( l_total == 0 ) return ETIR_SUCCESS;
  int64_t const l_blocks = ( l_total + 255 ) / 256;
  if( l_blocks > 0x7fffffffLL ) return fail( ETIR_UNDEFINED_ERROR, "split reduce: grid too large" );
  hipLaunchKernelGGL( split_reduce_kernel, dim3( (uint32_t) l_blocks ), dim3( 256 ), 0, stream, a );
  return ETIR_SUCCESS;
}

}  // namespace etir
