// Contractions with one short free side (kernel M or N of 2 to 64) and a
// long other side:
//   out[c][m][n] = touch( sum_k A[c][m][k] * B[c][n][k] ).
//
// Einsum-tree nodes of this shape (the einsum_benchmark MERA network has
// M = 11, N = 415800, K = 24 and M = 45, N = 196830, K = 11 on its longest
// chain) are bound by the long operand and the output, but on an MFMA tile
// most of every 64-row tile is padding, and with a short K each workgroup
// spends its life in one load round trip and the stores.  Here one thread
// owns one index of the long side and all outputs of the short side, in
// registers: the short operand is staged in LDS in chunks of 32 k (as fp32;
// every lane of a wave reads the same LDS address, a broadcast), the long
// operand is read once, by its own thread -- coalesced across threads when
// it is unit-stride along the long side, 16-byte vectors per thread when it
// is unit-stride along K.  Consecutive threads take consecutive long
// indices, so the stores of one short index coalesce where the output is
// unit-stride along the long side.
//
// Each output sums its K range in ascending k with one fp32 accumulator (the
// order of the matrix-vector kernel and of the reference's scalar backend,
// reference src/basic/binary/ContractionBackendScalar.cpp:30, once per K
// index of the loop nest of ContractionBackend.cpp:296-515); the touch
// kernels are applied once per output element as in the tiled kernels'
// epilogue (ContractionBackendTpp.cpp:84-163).
#include "etir_internal.h"
#include "contract_kernel.h"

#include <numeric>

namespace etir {

namespace {

template< typename T >
__device__ inline float sk_ld( T const * p, int64_t off );
template<>
__device__ inline float sk_ld< float >( float const * p, int64_t off ) { return p[off]; }
template<>
__device__ inline float sk_ld< uint16_t >( uint16_t const * p, int64_t off ) {
  return kern::bf16_to_f32( p[off] );
}

// four consecutive elements as one vector (16 bytes fp32, 8 bytes bf16)
template< typename T >
struct alignas( 4 * sizeof( T ) ) SkV4 { T v[4]; };

constexpr int kSkThreads = 256;
constexpr int kSkChunk   = 32;    // k per LDS chunk of the short operand

// SHORT_A: the short side is kernel M (operand A short, B long); else kernel
// N.  KVEC: the long operand is unit-stride along an affine K with every row
// offset a multiple of 4 elements and K % 4 == 0 (16-byte aligned rows).
template< typename T, int SMAX, bool SHORT_A, bool KAFF, bool KVEC >
__global__ __launch_bounds__( kSkThreads ) void contract_skinny_kernel( ContractArgs a ) {
  constexpr int KC = kSkChunk;
  // the short operand's chunk [KC][SMAX]; after the K loop, the block
  // store's staging [SC][kSkThreads + 1]
  constexpr int SC  = SMAX < 16 ? SMAX : 16;
  constexpr int RAW = KC * SMAX > SC * ( kSkThreads + 1 ) ? KC * SMAX : SC * ( kSkThreads + 1 );
  __shared__ float s_raw[RAW];
  float ( *s_op )[SMAX] = reinterpret_cast< float ( * )[SMAX] >( s_raw );
  // the short side's output and aux offsets, read from LDS in the epilogue:
  // a global table read between the stores would wait for every store
  // before it (one vector-memory counter for loads and stores)
  __shared__ int32_t s_oo[SMAX], s_ao[SMAX];

  int32_t const l_c     = blockIdx.y;
  int32_t const l_nlong = SHORT_A ? a.N : a.M;
  int32_t const l_nshrt = SHORT_A ? a.M : a.N;
  int32_t const l_i     = int32_t( blockIdx.x ) * kSkThreads + int32_t( threadIdx.x );
  bool const    l_in    = l_i < l_nlong;
  int32_t const l_ic    = l_in ? l_i : 0;     // threads past the long side load row 0, store nothing

  T const * l_ps = reinterpret_cast< T const * >( SHORT_A ? a.a : a.b ) + ( SHORT_A ? a.tc_a[l_c] : a.tc_b[l_c] );
  int32_t const * l_ts  = SHORT_A ? a.tm_a : a.tn_b;
  int32_t const * l_tks = SHORT_A ? a.tk_a : a.tk_b;
  int32_t const   l_sks = SHORT_A ? a.sk_a : a.sk_b;
  T const * l_pl = reinterpret_cast< T const * >( SHORT_A ? a.b : a.a )
                 + ( SHORT_A ? a.tc_b[l_c] + a.tn_b[l_ic] : a.tc_a[l_c] + a.tm_a[l_ic] );
  int32_t const * l_tkl = SHORT_A ? a.tk_b : a.tk_a;
  int32_t const   l_skl = SHORT_A ? a.sk_b : a.sk_a;
  auto koff_s = [&]( int32_t k ) -> int64_t { return KAFF ? int64_t( k ) * l_sks : int64_t( l_tks[k] ); };
  auto koff_l = [&]( int32_t k ) -> int64_t { return KAFF ? int64_t( k ) * l_skl : int64_t( l_tkl[k] ); };

  float l_acc[SMAX];
#pragma unroll
  for( int l_s = 0; l_s < SMAX; l_s++ ) l_acc[l_s] = 0.0f;

  // staging of the short operand: element e = t + 256 q (q < NI) of a chunk
  // is (k, s) = (e / SMAX, e % SMAX), so consecutive threads write
  // consecutive LDS words.  Thread t's short indices repeat with period
  // P = SMAX / gcd(256, SMAX) in q (1 where SMAX divides the workgroup, 3 for
  // SMAX 48), so it reads P row offsets once, and the NI loads of a chunk
  // are independent of each other and of the long operand's
  constexpr int NI = SMAX * KC / kSkThreads;
  constexpr int P  = SMAX / std::gcd( kSkThreads, SMAX );
  static_assert( ( SMAX * KC ) % kSkThreads == 0 && NI >= 1 && NI % P == 0, "skinny: SMAX x KC must fill the workgroup" );
  int32_t l_ss[P];
  int64_t l_srow[P];
#pragma unroll
  for( int l_p = 0; l_p < P; l_p++ ) {
    l_ss[l_p]   = ( int32_t( threadIdx.x ) + kSkThreads * l_p ) % SMAX;
    l_srow[l_p] = int64_t( l_ts[l_ss[l_p] < l_nshrt ? l_ss[l_p] : 0] );
  }
  if( threadIdx.x < SMAX ) {
    int32_t const * l_tso = SHORT_A ? a.tm_out : a.tn_out;
    int32_t const * l_tsa = SHORT_A ? a.tm_aux : a.tn_aux;
    bool const l_sok = int32_t( threadIdx.x ) < l_nshrt;
    s_oo[threadIdx.x] = l_sok ? l_tso[threadIdx.x] : 0;
    s_ao[threadIdx.x] = ( l_sok && a.aux != nullptr ) ? l_tsa[threadIdx.x] : 0;
  }
  __syncthreads();

  for( int32_t l_k0 = 0; l_k0 < a.K; l_k0 += KC ) {
    // the short operand's chunk, zero past the short side and past K
    float l_sv[NI];
#pragma unroll
    for( int l_q = 0; l_q < NI; l_q++ ) {
      int32_t const l_k = l_k0 + ( int32_t( threadIdx.x ) + kSkThreads * l_q ) / SMAX;
      l_sv[l_q] = ( l_ss[l_q % P] < l_nshrt && l_k < a.K ) ? sk_ld< T >( l_ps, l_srow[l_q % P] + koff_s( l_k ) )
                                                            : 0.0f;
    }
    // this thread's long-operand values of the chunk, all loads in flight together
    float l_x[KC];
    if constexpr( KVEC ) {
#pragma unroll
      for( int l_q = 0; l_q < KC / 4; l_q++ ) {
        int32_t const l_k = l_k0 + 4 * l_q;
        if( l_k < a.K ) {
          SkV4< T > const l_t = *reinterpret_cast< SkV4< T > const * >( l_pl + l_k );
#pragma unroll
          for( int l_j = 0; l_j < 4; l_j++ ) l_x[4 * l_q + l_j] = sk_ld< T >( l_t.v, l_j );
        }
        else {
#pragma unroll
          for( int l_j = 0; l_j < 4; l_j++ ) l_x[4 * l_q + l_j] = 0.0f;
        }
      }
    }
    else {
#pragma unroll
      for( int l_kk = 0; l_kk < KC; l_kk++ ) {
        l_x[l_kk] = ( l_k0 + l_kk < a.K ) ? sk_ld< T >( l_pl, koff_l( l_k0 + l_kk ) ) : 0.0f;
      }
    }
#pragma unroll
    for( int l_q = 0; l_q < NI; l_q++ ) s_raw[int( threadIdx.x ) + kSkThreads * l_q] = l_sv[l_q];
    __syncthreads();
    int32_t const l_kn = min( int32_t( KC ), a.K - l_k0 );
    // compile-time loops (accumulators and long-operand values stay in
    // registers; a partly unrolled loop would index them at run time)
    kern::static_for< KC >( [&]( auto kc ) __attribute__( ( always_inline ) ) {
      constexpr int l_kk = decltype( kc )::value;
      if( l_kk < l_kn ) {
        kern::static_for< SMAX >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
          constexpr int l_s = decltype( sc )::value;
          l_acc[l_s] = fmaf( s_op[l_kk][l_s], l_x[l_kk], l_acc[l_s] );
        } );
      }
    } );
    __syncthreads();
  }

  if( a.skinny_blk ) {
    // the output as [long][short], the short side unit-stride: the
    // workgroup's outputs are one block of (i1 - i0) * S elements, written in
    // chunks of SC short indices, each chunk in address order (runs of SC
    // elements S apart).  Element e of a chunk is long row t = e / ns, short
    // index sl = e - t * ns, with t = (e * ceil(2^16 / ns)) >> 16 (exact for
    // e < 4096 = 256 * 16, ns <= 16; 24-bit multiplies, full rate)
    constexpr uint32_t LD = kSkThreads + 1;      // LDS row stride: odd, successive short indices on other banks
    int32_t const  l_i0 = int32_t( blockIdx.x ) * kSkThreads;
    uint32_t const l_nl = uint32_t( min( l_i0 + kSkThreads, l_nlong ) - l_i0 );
    int64_t const  l_ob = a.tc_out[l_c] + int64_t( l_i0 ) * l_nshrt;
    kern::static_for< SMAX / SC >( [&]( auto cc ) __attribute__( ( always_inline ) ) {
      constexpr int l_s0 = decltype( cc )::value * SC;
      if( l_s0 >= l_nshrt ) return;
#pragma unroll
      for( int l_j = 0; l_j < SC; l_j++ ) {
        float l_v = l_acc[l_s0 + l_j];
        if( a.last_touch == ETIR_KTYPE_RELU ) l_v = fmaxf( l_v, 0.0f );
        s_raw[uint32_t( l_j ) * LD + threadIdx.x] = l_v;
      }
      __syncthreads();
      uint32_t const l_ns = uint32_t( min( SC, l_nshrt - l_s0 ) );
      uint32_t const l_m  = ( 65536u + l_ns - 1 ) / l_ns;
      uint32_t const l_n  = l_nl * l_ns;
      for( uint32_t l_e = threadIdx.x; l_e < l_n; l_e += kSkThreads ) {
        uint32_t const l_t  = __umul24( l_e, l_m ) >> 16;
        uint32_t const l_sl = l_e - __umul24( l_t, l_ns );
        float const l_v = s_raw[l_sl * LD + l_t];
        int64_t const l_off = l_ob + int64_t( __umul24( l_t, uint32_t( l_nshrt ) ) ) + l_s0 + l_sl;
        if( a.out_bf16 ) reinterpret_cast< uint16_t * >( a.out )[l_off] = kern::f32_to_bf16_rne( l_v );
        else             reinterpret_cast< float * >( a.out )[l_off] = l_v;
      }
      __syncthreads();
    } );
    return;
  }
  if( !l_in ) return;

  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux  = ( a.aux != nullptr ) && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
  int64_t const l_ob = a.tc_out[l_c] + ( SHORT_A ? a.tn_out[l_i] : a.tm_out[l_i] );
  int64_t const l_ab = l_need_aux ? a.tc_aux[l_c] + ( SHORT_A ? a.tn_aux[l_i] : a.tm_aux[l_i] ) : 0;
  // the touch kernels' loads of all short indices first, then the stores
  if( l_read_out || l_need_aux ) {
    kern::static_for< SMAX >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
      constexpr int l_s = decltype( sc )::value;
      if( l_s >= l_nshrt ) return;
      float l_v = l_acc[l_s];
      if( l_read_out ) {
        int64_t const l_off = l_ob + s_oo[l_s];
        l_v = ( a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.out )[l_off] )
                           : reinterpret_cast< float const * >( a.out )[l_off] ) + l_v;
      }
      if( l_need_aux ) {
        int64_t const l_aoff = l_ab + s_ao[l_s];
        float const l_aux = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.aux )[l_aoff] )
                                       : reinterpret_cast< float const * >( a.aux )[l_aoff];
        if( l_aux_first ) l_v = l_aux + l_v;
        if( a.last_touch == ETIR_KTYPE_ADD ) l_v = l_v + l_aux;
      }
      l_acc[l_s] = l_v;
    } );
  }
  kern::static_for< SMAX >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
    constexpr int l_s = decltype( sc )::value;
    if( l_s >= l_nshrt ) return;
    float l_v = l_acc[l_s];
    if( a.last_touch == ETIR_KTYPE_RELU ) l_v = fmaxf( l_v, 0.0f );
    int64_t const l_off = l_ob + s_oo[l_s];
    if( a.out_bf16 ) reinterpret_cast< uint16_t * >( a.out )[l_off] = kern::f32_to_bf16_rne( l_v );
    else             reinterpret_cast< float * >( a.out )[l_off] = l_v;
  } );
}

}  // namespace

int launch_contract_skinny( bool bf16_in, ContractArgs const & a, hipStream_t stream ) {
  bool const l_short_a = a.M <= a.N;
  int32_t const l_nshrt = l_short_a ? a.M : a.N;
  int32_t const l_nlong = l_short_a ? a.N : a.M;
  if( int64_t( a.C ) * l_nlong == 0 ) return ETIR_SUCCESS;
  if( l_nshrt > 64 ) return fail( ETIR_COMPILATION_FAILED, "skinny contraction: short side above 64" );
  if( a.C > 65535 ) return fail( ETIR_UNDEFINED_ERROR, "skinny contraction: more than 65535 C indices" );
  int64_t const l_esz = bf16_in ? 2 : 4;
  // vector loads of the long operand need its base address aligned to one vector
  void const * l_long_ptr = l_short_a ? a.b : a.a;
  bool const l_kvec = a.skinny_kvec && reinterpret_cast< uintptr_t >( l_long_ptr ) % uintptr_t( 4 * l_esz ) == 0;
  dim3 const l_grid( (uint32_t) ( ( l_nlong + kSkThreads - 1 ) / kSkThreads ), (uint32_t) a.C );
  bool const l_kaff = ( a.k_affine != 0 );
  auto go = [&]( auto t_c, auto smax_c, auto sa_c, auto kaff_c, auto kvec_c ) {
    typedef typename decltype( t_c )::type T;
    hipLaunchKernelGGL( ( contract_skinny_kernel< T, decltype( smax_c )::value, decltype( sa_c )::value,
                                                  decltype( kaff_c )::value, decltype( kvec_c )::value > ),
                        l_grid, dim3( kSkThreads ), 0, stream, a );
  };
  struct F32 { typedef float type; };
  struct BF16 { typedef uint16_t type; };
  auto pick_vec = [&]( auto t_c, auto smax_c, auto sa_c ) {
    // vector loads only with an affine K (the planner sets skinny_kvec only then)
    if( l_kvec )      go( t_c, smax_c, sa_c, std::true_type(), std::true_type() );
    else if( l_kaff ) go( t_c, smax_c, sa_c, std::true_type(), std::false_type() );
    else              go( t_c, smax_c, sa_c, std::false_type(), std::false_type() );
  };
  auto pick_side = [&]( auto t_c, auto smax_c ) {
    if( l_short_a ) pick_vec( t_c, smax_c, std::true_type() );
    else            pick_vec( t_c, smax_c, std::false_type() );
  };
  auto pick_smax = [&]( auto t_c ) {
    if(      l_nshrt <= 8 )  pick_side( t_c, std::integral_constant< int, 8 >() );
    else if( l_nshrt <= 16 ) pick_side( t_c, std::integral_constant< int, 16 >() );
    else if( l_nshrt <= 32 ) pick_side( t_c, std::integral_constant< int, 32 >() );
    else if( l_nshrt <= 48 ) pick_side( t_c, std::integral_constant< int, 48 >() );
    else                     pick_side( t_c, std::integral_constant< int, 64 >() );
  };
  if( bf16_in ) pick_smax( BF16() );
  else          pick_smax( F32() );
  return ETIR_SUCCESS;
}

}  // namespace etir
