// fp64 contraction kernel (tile f64_64x64x16) and its instantiations.
//
// Same contract as contract_kernel.h -- out[c][m][n] = touch( sum_k
// A[c][m][k] * B[c][n][k] ) over the planner's flattened C/M/N/K offset
// tables, every first/last-touch kernel of the reference's TPP backend
// (ContractionBackendTpp.cpp:127-163) applied once per output element -- for
// the reference's FP64 data type, on the fp64 matrix cores:
//   v_mfma_f64_16x16x4_f64: lane l supplies A[row l%16][k l/16] and
//   B[k l/16][col l%16]; the 16x16 result holds, in element r of lane l,
//   row 4*r + l/16 and column l%16 (measured with one-hot operands).
// Workgroup tile 64 x 64, K step 16, four waves in a 2 x 2 grid with 32 x 32
// each (2 x 2 MFMA blocks).  Operands go global -> registers -> LDS through
// the loaders of contract_kernel.h (16-byte vectors of two doubles along K or
// along M/N, or table gathers), double-buffered; the global loads of step
// k+1 are issued before the MFMAs of step k.  LDS layouts: [row][k] with
// pitch BK + 2 (the 64 lanes of one fragment read -- 16 rows x 4 k -- cover
// every bank exactly once per half-wave) or [k][row] with pitch
// KmPitch<64, 8> (two k rows of 16 consecutive doubles per half-wave, 128
// bytes apart modulo 256).
#include "contract_kernel.h"

namespace etir {
namespace kern {

typedef double f64x4 __attribute__( ( ext_vector_type( 4 ) ) );

template< int MODE, int R, int BK >
struct FragF64 {
  static constexpr int LDK = BK + 2;
  __device__ static inline double read( double const * lds, int row, int k ) {
    return lds[row * LDK + k];
  }
};

template< int R, int BK >
struct FragF64< LOAD_VEC_MN, R, BK > {
  static constexpr int PK = KmPitch< R, 8 >::value;
  __device__ static inline double read( double const * lds, int row, int k ) {
    return lds[k * PK + row];
  }
};

template< int MA, int MB, bool KAFF >
__global__ __launch_bounds__( 256, 1 )
void contract_f64_kernel( ContractArgs a ) {
  constexpr int BM = 64, BN = 64, BK = 16, T = 256;
  constexpr int SZA = LdsSize< 8, MA, BM, BK >::value;
  constexpr int SZB = LdsSize< 8, MB, BN, BK >::value;
  __shared__ __attribute__( ( aligned( 16 ) ) ) double l_lds_a[2][SZA];
  __shared__ __attribute__( ( aligned( 16 ) ) ) double l_lds_b[2][SZB];

  // XCD-aware order (consecutive workgroup ids go round-robin over the 8
  // XCDs: give each XCD one contiguous range), then groups of 8 tile rows
  int32_t const l_ntiles = a.tiles_m * a.tiles_n;
  int32_t const l_nblk   = gridDim.x;
  int32_t l_bid = blockIdx.x;
  if( ( l_nblk & 7 ) == 0 ) l_bid = ( l_bid & 7 ) * ( l_nblk >> 3 ) + ( l_bid >> 3 );
  int32_t const l_c      = a.c_inner ? l_bid % a.C : l_bid / l_ntiles;
  int32_t const l_tile   = a.c_inner ? l_bid / a.C : l_bid - l_c * l_ntiles;
  constexpr int32_t kGroupM = 8;
  int32_t const l_in_grp = kGroupM * a.tiles_n;
  int32_t const l_grp    = l_tile / l_in_grp;
  int32_t const l_fm     = l_grp * kGroupM;
  int32_t const l_gsz    = min( a.tiles_m - l_fm, kGroupM );
  int32_t const l_tm     = l_fm + ( l_tile - l_grp * l_in_grp ) % l_gsz;
  int32_t const l_tn     = ( l_tile - l_grp * l_in_grp ) / l_gsz;
  int32_t const l_m0     = l_tm * BM;
  int32_t const l_n0     = l_tn * BN;

  double const * l_a = reinterpret_cast< double const * >( a.a ) + a.tc_a[l_c];
  double const * l_b = reinterpret_cast< double const * >( a.b ) + a.tc_b[l_c];

  Loader< BM, BK, T, 8, MA > l_ld_a;
  Loader< BN, BK, T, 8, MB > l_ld_b;
  l_ld_a.init( a.tm_a, a.M, l_m0 );
  l_ld_b.init( a.tn_b, a.N, l_n0 );

  int const l_lane = threadIdx.x & 63;
  int const l_wave = threadIdx.x >> 6;
  int const l_wm   = l_wave >> 1;
  int const l_wn   = l_wave & 1;
  int const l_r16  = l_lane & 15;
  int const l_k4   = l_lane >> 4;

  f64x4 l_acc[2][2];
#pragma unroll
  for( int l_i = 0; l_i < 2; l_i++ )
#pragma unroll
    for( int l_j = 0; l_j < 2; l_j++ ) l_acc[l_i][l_j] = f64x4( 0.0 );

  int32_t const l_nk = ( a.K + BK - 1 ) / BK;
  if( l_nk > 0 ) {
    l_ld_a.template load< KAFF >( l_a, 0, a.K, a.tk_a, a.sk_a );
    l_ld_b.template load< KAFF >( l_b, 0, a.K, a.tk_b, a.sk_b );
    l_ld_a.store( l_lds_a[0] );
    l_ld_b.store( l_lds_b[0] );
    __syncthreads();

    for( int32_t l_kt = 0; l_kt < l_nk; l_kt++ ) {
      int const l_cur = l_kt & 1;
      bool const l_more = ( l_kt + 1 ) < l_nk;
      if( l_more ) {
        l_ld_a.template load< KAFF >( l_a, ( l_kt + 1 ) * BK, a.K, a.tk_a, a.sk_a );
        l_ld_b.template load< KAFF >( l_b, ( l_kt + 1 ) * BK, a.K, a.tk_b, a.sk_b );
      }
      double const * l_sa = l_lds_a[l_cur];
      double const * l_sb = l_lds_b[l_cur];
#pragma unroll
      for( int l_s = 0; l_s < BK / 4; l_s++ ) {
        int const l_k = 4 * l_s + l_k4;
        double l_fa[2], l_fb[2];
#pragma unroll
        for( int l_i = 0; l_i < 2; l_i++ ) {
          l_fa[l_i] = FragF64< MA, BM, BK >::read( l_sa, l_wm * 32 + l_i * 16 + l_r16, l_k );
          l_fb[l_i] = FragF64< MB, BN, BK >::read( l_sb, l_wn * 32 + l_i * 16 + l_r16, l_k );
        }
#pragma unroll
        for( int l_i = 0; l_i < 2; l_i++ )
#pragma unroll
          for( int l_j = 0; l_j < 2; l_j++ )
            l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f64_16x16x4f64( l_fa[l_i], l_fb[l_j], l_acc[l_i][l_j],
                                                                    0, 0, 0 );
      }
      if( l_more ) {
        l_ld_a.store( l_lds_a[l_cur ^ 1] );
        l_ld_b.store( l_lds_b[l_cur ^ 1] );
      }
      __syncthreads();
    }
  }

  // epilogue: touch kernels per element, 16 consecutive columns per 16 lanes
  int64_t const l_coff = a.tc_out[l_c];
  int64_t const l_coff_aux = ( a.aux != nullptr ) ? a.tc_aux[l_c] : 0;
  double * l_out = reinterpret_cast< double * >( a.out ) + l_coff;
  double const * l_aux = reinterpret_cast< double const * >( a.aux ) + l_coff_aux;
  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_aux_last  = ( a.last_touch == ETIR_KTYPE_ADD );
  bool const l_relu      = ( a.last_touch == ETIR_KTYPE_RELU );
#pragma unroll
  for( int l_j = 0; l_j < 2; l_j++ ) {
    int32_t const l_n = l_n0 + l_wn * 32 + l_j * 16 + l_r16;
    if( l_n >= a.N ) continue;
    int32_t const l_no = a.tn_out[l_n];
    int32_t const l_na = ( l_aux_first || l_aux_last ) ? a.tn_aux[l_n] : 0;
#pragma unroll
    for( int l_i = 0; l_i < 2; l_i++ ) {
#pragma unroll
      for( int l_r = 0; l_r < 4; l_r++ ) {
        int32_t const l_m = l_m0 + l_wm * 32 + l_i * 16 + 4 * l_r + l_k4;
        if( l_m >= a.M ) continue;
        int64_t const l_off = int64_t( a.tm_out[l_m] ) + l_no;
        double l_v = l_acc[l_i][l_j][l_r];
        double l_x = 0.0;
        if( l_aux_first || l_aux_last ) l_x = l_aux[ int64_t( a.tm_aux[l_m] ) + l_na ];
        if( l_read_out ) l_v = l_out[l_off] + l_v;
        if( l_aux_first ) l_v = l_x + l_v;
        if( l_relu ) l_v = fmax( l_v, 0.0 );
        else if( l_aux_last ) l_v = l_v + l_x;
        l_out[l_off] = l_v;
      }
    }
  }
}

}  // namespace kern

int launch_contract_f64_64x64( int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                               uint32_t grid, hipStream_t stream ) {
  return with_load_modes( ma, mb, kaff, [&]( auto i_ma, auto i_mb, auto i_kaff ) {
    hipLaunchKernelGGL( ( kern::contract_f64_kernel< decltype( i_ma )::value, decltype( i_mb )::value,
                                                     decltype( i_kaff )::value > ),
                        dim3( grid ), dim3( 256 ), 0, stream, a );
    return int( ETIR_SUCCESS );
  } );
}

}  // namespace etir
