// fp32 contraction for few output tiles and a moderate K, both operands
// K-contiguous: the K range is split over the waves of ONE workgroup, so the
// partial sums meet in LDS instead of in a workspace in memory.
//
//   out[c][m][n] = touch( sum_k A[c][m][k] * B[c][n][k] )
//
// One workgroup of W waves per 32 x 32 output tile.  Wave w computes the whole
// tile over its own range of K (KW consecutive k, a multiple of 16), loading
// its operands straight into registers -- lane (r, q) of the wave reads the
// 16 bytes A[m0 + r][k + 4q .. k + 4q + 3] (and likewise B), which are exactly
// the fp32 values v_mfma_f32_16x16x4f32 wants from that lane for four MFMAs
// (MFMA j of a group takes element j; its four k rows are the lanes' q) --
// so no LDS staging and no barrier in the main loop.  Four lanes read 64
// contiguous bytes of one row (with 32 x 32 x 2 MFMAs, whose lanes split k
// only two ways, a load instruction would touch twice as many cache lines).  The W partial tiles are
// then added in LDS in wave order (a fixed order: results are reproducible)
// and the first/last-touch kernels applied once per output element, with the
// semantics of reference src/basic/binary/ContractionBackendTpp.cpp:84-163
// (ZERO/COPY/ADD first touch, RELU/ADD last touch, aux broadcasts).
//
// Where split-K sends S partial tiles through memory and a second kernel
// (reference loop nest: first/last touch at the K-loop boundaries,
// src/basic/binary/ContractionBackend.cpp:296-348), here one launch moves the
// operands once and the output once.
#include "contract_kernel.h"

namespace etir {

namespace {

using kern::f32x4;

constexpr int kTile = 32;     // output tile is kTile x kTile
constexpr int kChunk = 64;    // k per register batch (16 loads of 16 bytes in flight)
constexpr int kPitch = kTile + 1;

template< int W >
__global__ __launch_bounds__( 64 * W )
void contract_kwave_kernel( ContractArgs a, int32_t kw ) {
  constexpr int T = 64 * W;
  __shared__ float l_part[W][kTile * kPitch];

  // tile order as in the other contraction kernels: XCD-contiguous ranges,
  // groups of 8 tile rows
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
  int32_t const l_m0     = ( l_fm + ( l_tile - l_grp * l_in_grp ) % l_gsz ) * kTile;
  int32_t const l_n0     = ( ( l_tile - l_grp * l_in_grp ) / l_gsz ) * kTile;

  int const l_lane = threadIdx.x & 63;
  int const l_wave = __builtin_amdgcn_readfirstlane( threadIdx.x >> 6 );
  int const l_r    = l_lane & 15;      // row (A) / column (B) within a 16-row half
  int const l_q    = l_lane >> 4;      // k quarter

  // C offsets: with one C value (no C dims) every table holds the single
  // offset 0, so no table is read -- a memory round trip less before the
  // first operand load and before the stores
  bool const l_one_c = ( a.C == 1 );
  int64_t const l_ca = l_one_c ? 0 : a.tc_a[l_c];
  int64_t const l_cb = l_one_c ? 0 : a.tc_b[l_c];
  int64_t const l_coff = l_one_c ? 0 : a.tc_out[l_c];

  // this lane's rows of A / columns of B (two 16-row halves of the tile) at
  // k = 0 (K is affine: k * sk); an affine row table is not read, which saves
  // a memory round trip before the first operand load
  float const * l_pa[2];
  float const * l_pb[2];
  bool l_mok[2], l_nok[2];
#pragma unroll
  for( int l_x = 0; l_x < 2; l_x++ ) {
    int32_t const l_m = l_m0 + 16 * l_x + l_r;
    int32_t const l_n = l_n0 + 16 * l_x + l_r;
    l_mok[l_x] = l_m < a.M;
    l_nok[l_x] = l_n < a.N;
    int64_t const l_ra = !l_mok[l_x] ? 0 : ( a.sm_a >= 0 ? int64_t( l_m ) * a.sm_a : a.tm_a[l_m] );
    int64_t const l_rb = !l_nok[l_x] ? 0 : ( a.sn_b >= 0 ? int64_t( l_n ) * a.sn_b : a.tn_b[l_n] );
    l_pa[l_x] = reinterpret_cast< float const * >( a.a ) + l_ca + l_ra;
    l_pb[l_x] = reinterpret_cast< float const * >( a.b ) + l_cb + l_rb;
  }

  // output offsets of the elements this thread stores at the end (rows
  // threadIdx / 32 + (T / 32) u, column threadIdx % 32): read now, so the
  // loads overlap the operand loads instead of following the MFMAs
  constexpr int NU = ( kTile * kTile + T - 1 ) / T;
  int const l_scol = threadIdx.x % kTile;
  int32_t const l_sn = min( l_n0 + l_scol, a.N - 1 );
  int64_t const l_so_n = a.sn_out >= 0 ? int64_t( l_sn ) * a.sn_out : a.tn_out[l_sn];
  int64_t l_so_m[NU];
#pragma unroll
  for( int l_u = 0; l_u < NU; l_u++ ) {
    int32_t const l_sm = min( l_m0 + int( threadIdx.x ) / kTile + ( T / kTile ) * l_u, a.M - 1 );
    l_so_m[l_u] = a.sm_out >= 0 ? int64_t( l_sm ) * a.sm_out : a.tm_out[l_sm];
  }

  // v_mfma_f32_16x16x4f32 over the 2 x 2 blocks of 16 x 16: lane (r, q)
  // reads the 16 bytes A[row r][k + 4q .. k + 4q + 3] (four lanes cover 64
  // contiguous bytes of a row), and MFMA j of a 16-k group takes element j,
  // i.e. k + 4q + j for the MFMA's k index q
  int32_t const l_k0 = l_wave * kw;
  int32_t const l_k1 = min( l_k0 + kw, a.K );
  f32x4 l_acc[2][2];
#pragma unroll
  for( int l_x = 0; l_x < 2; l_x++ )
#pragma unroll
    for( int l_y = 0; l_y < 2; l_y++ ) l_acc[l_x][l_y] = f32x4( 0.0f );
  for( int32_t l_kc = l_k0; l_kc < l_k1; l_kc += kChunk ) {
    // one batch: up to kChunk / 16 groups of 16 k, all loads issued before any MFMA
    int32_t const l_ng = min( kChunk, l_k1 - l_kc ) / 16;
    f32x4 l_va[kChunk / 16][2], l_vb[kChunk / 16][2];
#pragma unroll
    for( int l_g = 0; l_g < kChunk / 16; l_g++ ) {
      int32_t const l_k = l_kc + 16 * l_g + 4 * l_q;
#pragma unroll
      for( int l_x = 0; l_x < 2; l_x++ ) {
        l_va[l_g][l_x] = ( l_g < l_ng && l_mok[l_x] )
                       ? *reinterpret_cast< f32x4 const * >( l_pa[l_x] + int64_t( l_k ) * a.sk_a ) : f32x4( 0.0f );
        l_vb[l_g][l_x] = ( l_g < l_ng && l_nok[l_x] )
                       ? *reinterpret_cast< f32x4 const * >( l_pb[l_x] + int64_t( l_k ) * a.sk_b ) : f32x4( 0.0f );
      }
    }
#pragma unroll
    for( int l_g = 0; l_g < kChunk / 16; l_g++ ) {
      if( l_g < l_ng ) {
#pragma unroll
        for( int l_j = 0; l_j < 4; l_j++ )
#pragma unroll
          for( int l_x = 0; l_x < 2; l_x++ )
#pragma unroll
            for( int l_y = 0; l_y < 2; l_y++ )
              l_acc[l_x][l_y] = __builtin_amdgcn_mfma_f32_16x16x4f32( l_va[l_g][l_x][l_j], l_vb[l_g][l_y][l_j],
                                                                      l_acc[l_x][l_y], 0, 0, 0 );
      }
    }
  }

  // partial tile of this wave -> LDS: element i of lane (r, q) in block
  // (x, y) is row 16 x + 4 q + i, column 16 y + r
#pragma unroll
  for( int l_x = 0; l_x < 2; l_x++ )
#pragma unroll
    for( int l_y = 0; l_y < 2; l_y++ )
#pragma unroll
      for( int l_i = 0; l_i < 4; l_i++ )
        l_part[l_wave][( 16 * l_x + 4 * l_q + l_i ) * kPitch + 16 * l_y + l_r] = l_acc[l_x][l_y][l_i];
  __syncthreads();

  // sum of the partial tiles in wave order, touch kernels, store; consecutive
  // threads take consecutive columns (the output's unit-stride index)
  bool const l_read_out  = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux  = ( a.aux != nullptr ) && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
  int64_t const l_caux = ( l_need_aux && !l_one_c ) ? a.tc_aux[l_c] : 0;
#pragma unroll
  for( int l_u = 0; l_u < NU; l_u++ ) {
    int const l_e = threadIdx.x + T * l_u;
    if( l_e >= kTile * kTile ) break;
    int const l_row = l_e / kTile;
    int const l_col = l_e % kTile;
    int32_t const l_mm = l_m0 + l_row;
    int32_t const l_nn = l_n0 + l_col;
    if( l_mm >= a.M || l_nn >= a.N ) continue;
    float l_v = 0.0f;
#pragma unroll
    for( int l_w = 0; l_w < W; l_w++ ) l_v += l_part[l_w][l_row * kPitch + l_col];
    int64_t const l_off = l_coff + l_so_m[l_u] + l_so_n;
    float l_aux = 0.0f;
    if( l_need_aux ) {
      int64_t const l_aoff = l_caux + a.tm_aux[l_mm] + a.tn_aux[l_nn];
      l_aux = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.aux )[l_aoff] )
                         : reinterpret_cast< float const * >( a.aux )[l_aoff];
    }
    if( l_read_out ) {
      float const l_old = a.out_bf16 ? kern::bf16_to_f32( reinterpret_cast< uint16_t const * >( a.out )[l_off] )
                                     : reinterpret_cast< float const * >( a.out )[l_off];
      l_v = l_old + l_v;
    }
    if( l_aux_first ) l_v = l_aux + l_v;
    if( a.last_touch == ETIR_KTYPE_RELU ) l_v = fmaxf( l_v, 0.0f );
    else if( a.last_touch == ETIR_KTYPE_ADD ) l_v = l_v + l_aux;
    if( a.out_bf16 ) reinterpret_cast< uint16_t * >( a.out )[l_off] = kern::f32_to_bf16_rne( l_v );
    else             reinterpret_cast< float * >( a.out )[l_off] = l_v;
  }
}

}  // namespace

// waves: 4, 8 or 16; kw: k per wave (multiple of 16, kw * waves >= K)
int launch_contract_kwave( int32_t waves, int32_t kw, ContractArgs const & a, uint32_t grid,
                           hipStream_t stream ) {
  if( kw <= 0 || kw % 16 != 0 || int64_t( kw ) * waves < a.K ) {
    return fail( ETIR_UNDEFINED_ERROR, "kwave: k per wave must be a positive multiple of 16 covering K" );
  }
  if( waves == 4 ) {
    hipLaunchKernelGGL( contract_kwave_kernel< 4 >, dim3( grid ), dim3( 256 ), 0, stream, a, kw );
  }
  else if( waves == 8 ) {
    hipLaunchKernelGGL( contract_kwave_kernel< 8 >, dim3( grid ), dim3( 512 ), 0, stream, a, kw );
  }
  else if( waves == 16 ) {
    hipLaunchKernelGGL( contract_kwave_kernel< 16 >, dim3( grid ), dim3( 1024 ), 0, stream, a, kw );
  }
  else {
    return fail( ETIR_UNDEFINED_ERROR, "kwave: 4, 8 or 16 waves" );
  }
  return ETIR_SUCCESS;
}

}  // namespace etir
