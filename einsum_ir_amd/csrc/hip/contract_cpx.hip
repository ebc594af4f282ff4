// Complex contraction kernels (tiles cpx_f32_64x64x16, cpx_f64_64x64x16).
//
// The reference's CPX_MADD (run by its BLAS backend,
// reference src/backend/BinaryContractionBlas.cpp:68-85, and used by every
// contraction node of a complex einsum expression, EinsumExpression.cpp:251-252):
// one loop of the IR is the complex dimension (size 2: real part at offset 0,
// imaginary part at the loop's stride, per tensor); all other loops form the
// flattened C/M/N/K offset tables of contract_kernel.h.  Per output element
//   out_re = sum_k ( A_re B_re - A_im B_im )
//   out_im = sum_k ( A_re B_im + A_im B_re )
// with first touch ZERO / CPX_ZERO (start from 0) or UNDEFINED (add to the
// output's old value).
//
// Structure: tile 64 x 64, K step 16, four waves in a 2 x 2 grid with 32 x 32
// each; four operand tiles (A re/im, B re/im) go global -> registers -> LDS
// through the loaders of contract_kernel.h, double-buffered.  MFMA with 16 x 16
// blocks and 4 k per instruction for both types:
//   fp32 v_mfma_f32_16x16x4_f32: lane l feeds A[l%16][l/16], B[l/16][l%16];
//        element r of the result is row 4*(l/16) + r, column l%16;
//   fp64 v_mfma_f64_16x16x4_f64: same operands; element r is row 4*r + l/16
// (both layouts measured with one-hot operands).  Each complex block product
// takes four MFMAs into two accumulators; the A_im fragment is negated in
// registers for the real part.
#include "contract_kernel.h"

namespace etir {
namespace kern {

typedef double f64x4 __attribute__( ( ext_vector_type( 4 ) ) );

template< typename T > struct Mfma16;
template<> struct Mfma16< float > {
  typedef f32x4 V;
  __device__ static inline V mma( float a, float b, V c ) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32( a, b, c, 0, 0, 0 );
  }
  __device__ static inline int row( int r, int lane_group ) { return 4 * lane_group + r; }
};
template<> struct Mfma16< double > {
  typedef f64x4 V;
  __device__ static inline V mma( double a, double b, V c ) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64( a, b, c, 0, 0, 0 );
  }
  __device__ static inline int row( int r, int lane_group ) { return 4 * r + lane_group; }
};

template< typename T, int MODE, int R, int BK >
struct FragCpx {
  static constexpr int LDK = BK + 16 / int( sizeof( T ) );
  __device__ static inline T read( T const * lds, int row, int k ) { return lds[row * LDK + k]; }
};
template< typename T, int R, int BK >
struct FragCpx< T, LOAD_VEC_MN, R, BK > {
  static constexpr int PK = KmPitch< R, int( sizeof( T ) ) >::value;
  __device__ static inline T read( T const * lds, int row, int k ) { return lds[k * PK + row]; }
};

template< typename T, int MA, int MB, bool KAFF >
__global__ __launch_bounds__( 256, 1 )
void contract_cpx_kernel( ContractArgs a ) {
  constexpr int BM = 64, BN = 64, BK = 16, T_ = 256, ESZ = int( sizeof( T ) );
  constexpr int SZA = LdsSize< ESZ, MA, BM, BK >::value;
  constexpr int SZB = LdsSize< ESZ, MB, BN, BK >::value;
  // [buffer][re/im][elements]
  __shared__ __attribute__( ( aligned( 16 ) ) ) T l_lds_a[2][2][SZA];
  __shared__ __attribute__( ( aligned( 16 ) ) ) T l_lds_b[2][2][SZB];
  typedef Mfma16< T > MF;
  typedef typename MF::V V;

  int32_t const l_ntiles = a.tiles_m * a.tiles_n;
  int32_t const l_nblk   = gridDim.x;
  int32_t l_bid = blockIdx.x;
  if( ( l_nblk & 7 ) == 0 ) l_bid = ( l_bid & 7 ) * ( l_nblk >> 3 ) + ( l_bid >> 3 );
  int32_t const l_c      = a.c_inner ? l_bid % a.C : l_bid / l_ntiles;
  int32_t const l_tile   = a.c_inner ? l_bid / a.C : l_bid - l_c * l_ntiles;
  int32_t const l_tm     = l_tile / a.tiles_n;
  int32_t const l_tn     = l_tile - l_tm * a.tiles_n;
  int32_t const l_m0     = l_tm * BM;
  int32_t const l_n0     = l_tn * BN;

  T const * l_a_re = reinterpret_cast< T const * >( a.a ) + a.tc_a[l_c];
  T const * l_b_re = reinterpret_cast< T const * >( a.b ) + a.tc_b[l_c];
  T const * l_a_im = l_a_re + a.cpx_a;
  T const * l_b_im = l_b_re + a.cpx_b;

  // the loaders' per-thread row offsets are the same for both parts
  Loader< BM, BK, T_, ESZ, MA > l_ld_ar, l_ld_ai;
  Loader< BN, BK, T_, ESZ, MB > l_ld_br, l_ld_bi;
  l_ld_ar.init( a.tm_a, a.M, l_m0 );
  l_ld_ai.init( a.tm_a, a.M, l_m0 );
  l_ld_br.init( a.tn_b, a.N, l_n0 );
  l_ld_bi.init( a.tn_b, a.N, l_n0 );

  int const l_lane = threadIdx.x & 63;
  int const l_wave = threadIdx.x >> 6;
  int const l_wm   = l_wave >> 1;
  int const l_wn   = l_wave & 1;
  int const l_r16  = l_lane & 15;
  int const l_g    = l_lane >> 4;

  V l_re[2][2], l_im[2][2];
#pragma unroll
  for( int l_i = 0; l_i < 2; l_i++ )
#pragma unroll
    for( int l_j = 0; l_j < 2; l_j++ ) {
      l_re[l_i][l_j] = V( T( 0 ) );
      l_im[l_i][l_j] = V( T( 0 ) );
    }

  auto load = [&]( int32_t k0 ) __attribute__( ( always_inline ) ) {
    l_ld_ar.template load< KAFF >( l_a_re, k0, a.K, a.tk_a, a.sk_a );
    l_ld_ai.template load< KAFF >( l_a_im, k0, a.K, a.tk_a, a.sk_a );
    l_ld_br.template load< KAFF >( l_b_re, k0, a.K, a.tk_b, a.sk_b );
    l_ld_bi.template load< KAFF >( l_b_im, k0, a.K, a.tk_b, a.sk_b );
  };
  auto store = [&]( int buf ) __attribute__( ( always_inline ) ) {
    l_ld_ar.store( l_lds_a[buf][0] );
    l_ld_ai.store( l_lds_a[buf][1] );
    l_ld_br.store( l_lds_b[buf][0] );
    l_ld_bi.store( l_lds_b[buf][1] );
  };

  int32_t const l_nk = ( a.K + BK - 1 ) / BK;
  if( l_nk > 0 ) {
    load( 0 );
    store( 0 );
    __syncthreads();
    for( int32_t l_kt = 0; l_kt < l_nk; l_kt++ ) {
      int const l_cur = l_kt & 1;
      bool const l_more = ( l_kt + 1 ) < l_nk;
      if( l_more ) load( ( l_kt + 1 ) * BK );
#pragma unroll
      for( int l_s = 0; l_s < BK / 4; l_s++ ) {
        int const l_k = 4 * l_s + l_g;
        T l_ar[2], l_ai[2], l_nai[2], l_br[2], l_bi[2];
#pragma unroll
        for( int l_i = 0; l_i < 2; l_i++ ) {
          int const l_ra = l_wm * 32 + l_i * 16 + l_r16;
          int const l_rb = l_wn * 32 + l_i * 16 + l_r16;
          l_ar[l_i]  = FragCpx< T, MA, BM, BK >::read( l_lds_a[l_cur][0], l_ra, l_k );
          l_ai[l_i]  = FragCpx< T, MA, BM, BK >::read( l_lds_a[l_cur][1], l_ra, l_k );
          l_br[l_i]  = FragCpx< T, MB, BN, BK >::read( l_lds_b[l_cur][0], l_rb, l_k );
          l_bi[l_i]  = FragCpx< T, MB, BN, BK >::read( l_lds_b[l_cur][1], l_rb, l_k );
          l_nai[l_i] = -l_ai[l_i];
        }
#pragma unroll
        for( int l_i = 0; l_i < 2; l_i++ )
#pragma unroll
          for( int l_j = 0; l_j < 2; l_j++ ) {
            l_re[l_i][l_j] = MF::mma( l_ar[l_i],  l_br[l_j], l_re[l_i][l_j] );
            l_re[l_i][l_j] = MF::mma( l_nai[l_i], l_bi[l_j], l_re[l_i][l_j] );
            l_im[l_i][l_j] = MF::mma( l_ar[l_i],  l_bi[l_j], l_im[l_i][l_j] );
            l_im[l_i][l_j] = MF::mma( l_ai[l_i],  l_br[l_j], l_im[l_i][l_j] );
          }
      }
      if( l_more ) store( l_cur ^ 1 );
      __syncthreads();
    }
  }

  // epilogue: real and imaginary part of every element of the wave's blocks
  T * l_out = reinterpret_cast< T * >( a.out ) + a.tc_out[l_c];
  bool const l_acc_out = ( a.first_touch == ETIR_KTYPE_UNDEFINED );
#pragma unroll
  for( int l_j = 0; l_j < 2; l_j++ ) {
    int32_t const l_n = l_n0 + l_wn * 32 + l_j * 16 + l_r16;
    if( l_n >= a.N ) continue;
    int64_t const l_no = a.tn_out[l_n];
#pragma unroll
    for( int l_i = 0; l_i < 2; l_i++ ) {
#pragma unroll
      for( int l_r = 0; l_r < 4; l_r++ ) {
        int32_t const l_m = l_m0 + l_wm * 32 + l_i * 16 + MF::row( l_r, l_g );
        if( l_m >= a.M ) continue;
        int64_t const l_off = int64_t( a.tm_out[l_m] ) + l_no;
        T l_vr = l_re[l_i][l_j][l_r];
        T l_vi = l_im[l_i][l_j][l_r];
        if( l_acc_out ) {
          l_vr = l_out[l_off] + l_vr;
          l_vi = l_out[l_off + a.cpx_out] + l_vi;
        }
        l_out[l_off] = l_vr;
        l_out[l_off + a.cpx_out] = l_vi;
      }
    }
  }
}

template< typename T >
int launch_cpx_typed( int32_t ma, int32_t mb, bool kaff, ContractArgs const & a, uint32_t grid,
                      hipStream_t stream ) {
  return with_load_modes( ma, mb, kaff, [&]( auto i_ma, auto i_mb, auto i_kaff ) {
    hipLaunchKernelGGL( ( contract_cpx_kernel< T, decltype( i_ma )::value, decltype( i_mb )::value,
                                               decltype( i_kaff )::value > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return int( ETIR_SUCCESS );
  } );
}

}  // namespace kern

int launch_contract_cpx( bool f64, int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                         uint32_t grid, hipStream_t stream ) {
  return f64 ? kern::launch_cpx_typed< double >( ma, mb, kaff, a, grid, stream )
             : kern::launch_cpx_typed< float >( ma, mb, kaff, a, grid, stream );
}

}  // namespace etir
