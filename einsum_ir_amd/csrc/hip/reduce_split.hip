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

}  // namespace

int launch_split_reduce( SplitReduceArgs const & a, hipStream_t stream ) {
  int64_t const l_total = int64_t( a.C ) * a.M * a.N;
  if( l_total == 0 ) return ETIR_SUCCESS;
  int64_t const l_blocks = ( l_total + 255 ) / 256;
  if( l_blocks > 0x7fffffffLL ) return fail( ETIR_UNDEFINED_ERROR, "split reduce: grid too large" );
  hipLaunchKernelGGL( split_reduce_kernel, dim3( (uint32_t) l_blocks ), dim3( 256 ), 0, stream, a );
  return ETIR_SUCCESS;
}

}  // namespace etir
