// fp32 contraction kernel with direct-to-LDS operand loads.
//
// Same contraction and first/last-touch epilogue as contract_kernel.h
//   out[c][m][n] = touch( sum_k A[c][m][k] * B[c][n][k] )
// (reference src/basic/binary/ContractionBackendTpp.cpp:127-163 for the touch
// kernels), for large fp32 contractions with 16-byte vector operands:
// 128 x 128 tiles, k step 32, 8 waves of 32 x 64
// (v_mfma_f32_32x32x2_f32), two LDS stages of 32 KB (two workgroups per CU,
// four waves per SIMD).
//
// The operands go global -> LDS with buffer_load_dwordx4 ... lds (dma16 of
// contract_dma.h): no staging registers, no ds_write, and no wait for the
// global loads in the middle of a k step.  In the register-staged kernel
// those cost about a tenth of the time at 4096^3 (measured by taking the
// loads, then the LDS stores, out of a timing copy: 80.6 -> 86 -> 91 % of
// peak).  Step t issues the loads of step t + 1 into the other stage between
// the MFMAs of its first fragment step and ends with one wait + barrier.
// Rows past M/N and k past K read zeros through the buffer range check.
// A K that is not one affine index (K <= 1024) takes its offsets from the
// plan's K tables, staged in LDS once per workgroup.
//
// LDS layouts per stage, written one KiB per DMA instruction (lane i at 16 i):
// VEC_MN (16-byte runs along the rows): [k][R] fp32, R * 4 bytes per k row;
//   the 16-byte segment g (rows 4g .. 4g+3) of k row k is stored at segment
//   g ^ swz_f32_mn(k).  A fragment read (4 bytes: row lane % 32, k rows
//   k0 + 4 (lane / 32) + e) has its two half-waves 4 k rows apart; the
//   swizzle puts their segments in opposite halves of the 256-byte bank
//   window, so the 64 lanes hit 64 banks.
// VEC_K (16-byte runs along K): [R][BK] fp32, 128 bytes per row, segment g
//   (4 k) of row r stored at g ^ swz_k(r) -- the byte layout of the bf16
//   VEC_K stage of contract_dma.h; a fragment is one ds_read_b128 of segment
//   2 s + lane / 32.
#include "contract_dma.h"

namespace etir {
namespace kern {

// longest K whose offset tables the kernel stages in LDS (2 x 4 KB)
constexpr int kF32DmaMaxTableK = 1024;

__device__ inline uint32_t swz_f32_mn( int k ) {
  return uint32_t( ( k & 4 ) << 1 );
}

template< int R, int BK, int W, int MODE >
struct F32DmaLoader;

template< int R, int BK, int W >
struct F32DmaLoader< R, BK, W, LOAD_VEC_MN > {
  static constexpr int SEGS  = R / 4;          // 16-byte segments per k row
  static constexpr int KPC   = 64 / SEGS;      // k rows per KiB chunk
  static constexpr int NCH   = BK / KPC;       // chunks per stage
  static constexpr int NJ    = NCH / W;        // chunks per wave
  static constexpr int STAGE_BYTES = BK * R * 4;
  static_assert( SEGS >= 16 && SEGS <= 64 && 64 % SEGS == 0, "fp32 VEC_MN DMA: R must be 64..256" );
  static_assert( NCH % W == 0 && NJ >= 1, "fp32 VEC_MN DMA: chunks must divide over the waves" );

  uint32_t m_off[NJ];   // byte offset of the lane's segment at k step 0 (kDmaOob: row outside)
  int32_t  m_kk[NJ];    // k row of the lane's segment within the step

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0, int32_t sk,
                               int wave, int lane ) {
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      int const l_kk  = ( wave * NJ + l_j ) * KPC + lane / SEGS;
      int const l_g   = ( lane % SEGS ) ^ int( swz_f32_mn( l_kk ) );
      int32_t const l_row = row0 + 4 * l_g;
      m_kk[l_j]  = l_kk;
      m_off[l_j] = ( l_row < rows ) ? uint32_t( 4 * ( tab_rows[l_row] + l_kk * sk ) ) : kDmaOob;
    }
  }

  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline void issue_one( i32x4 rsrc, uint32_t lds_stage, int wave,
                                                                       int32_t k0, int32_t K,
                                                                       uint32_t kstep_bytes ) {
    uint32_t const l_off = ( k0 + m_kk[J] < K ) ? m_off[J] + kstep_bytes : kDmaOob;
    dma16( rsrc, l_off, lds_stage + ( wave * NJ + J ) * 1024 );
  }

  // K through an offset table (staged in LDS): m_off holds the row part only
  __device__ inline void init_tab( int32_t const * tab_rows, int32_t rows, int32_t row0, int wave, int lane ) {
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      int const l_kk  = ( wave * NJ + l_j ) * KPC + lane / SEGS;
      int const l_g   = ( lane % SEGS ) ^ int( swz_f32_mn( l_kk ) );
      int32_t const l_row = row0 + 4 * l_g;
      m_kk[l_j]  = l_kk;
      m_off[l_j] = ( l_row < rows ) ? uint32_t( 4 * tab_rows[l_row] ) : kDmaOob;
    }
  }
  // table entry of the lane's k row in step k0 (0 past K: the load is out of range anyway)
  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline int32_t tab_entry( int32_t const * tab_k, int32_t k0,
                                                                         int32_t K ) const {
    int32_t const l_k = k0 + m_kk[J];
    return tab_k[l_k < K ? l_k : 0];
  }
  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline void issue_tab( i32x4 rsrc, uint32_t lds_stage, int wave,
                                                                       int32_t k0, int32_t K, int32_t koff ) {
    uint32_t const l_off = ( k0 + m_kk[J] < K ) ? m_off[J] + uint32_t( 4 * koff ) : kDmaOob;
    dma16( rsrc, l_off, lds_stage + ( wave * NJ + J ) * 1024 );
  }
};

template< int R, int BK, int W >
struct F32DmaLoader< R, BK, W, LOAD_VEC_K > {
  static constexpr int SEGS  = BK / 4;         // 16-byte segments per row
  static constexpr int RPC   = 64 / SEGS;      // rows per KiB chunk
  static constexpr int NCH   = R / RPC;
  static constexpr int NJ    = NCH / W;
  static constexpr int STAGE_BYTES = BK * R * 4;
  static_assert( SEGS == 8, "fp32 VEC_K DMA: BK must be 32" );
  static_assert( NCH % W == 0 && NJ >= 1, "fp32 VEC_K DMA: chunks must divide over the waves" );

  uint32_t m_off[NJ];
  int32_t  m_kl[NJ];   // first k of the lane's segment within the step

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0, int32_t sk,
                               int wave, int lane ) {
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      int const l_r   = ( wave * NJ + l_j ) * RPC + lane / SEGS;
      int const l_g   = ( lane % SEGS ) ^ int( swz_k( l_r ) );
      int32_t const l_row = row0 + l_r;
      m_kl[l_j]  = 4 * l_g;
      m_off[l_j] = ( l_row < rows ) ? uint32_t( 4 * ( tab_rows[l_row] + 4 * l_g * sk ) ) : kDmaOob;
    }
  }

  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline void issue_one( i32x4 rsrc, uint32_t lds_stage, int wave,
                                                                       int32_t k0, int32_t K,
                                                                       uint32_t kstep_bytes ) {
    uint32_t const l_off = ( k0 + m_kl[J] < K ) ? m_off[J] + kstep_bytes : kDmaOob;
    dma16( rsrc, l_off, lds_stage + ( wave * NJ + J ) * 1024 );
  }

  // K through an offset table: the planner's VEC_K mode guarantees runs of
  // 4 consecutive k at consecutive offsets, so the lane's 4 k start at
  // tab_k[k0 + 4g]
  __device__ inline void init_tab( int32_t const * tab_rows, int32_t rows, int32_t row0, int wave, int lane ) {
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      int const l_r   = ( wave * NJ + l_j ) * RPC + lane / SEGS;
      int const l_g   = ( lane % SEGS ) ^ int( swz_k( l_r ) );
      int32_t const l_row = row0 + l_r;
      m_kl[l_j]  = 4 * l_g;
      m_off[l_j] = ( l_row < rows ) ? uint32_t( 4 * tab_rows[l_row] ) : kDmaOob;
    }
  }
  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline int32_t tab_entry( int32_t const * tab_k, int32_t k0,
                                                                         int32_t K ) const {
    int32_t const l_k = k0 + m_kl[J];
    return tab_k[l_k < K ? l_k : 0];
  }
  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline void issue_tab( i32x4 rsrc, uint32_t lds_stage, int wave,
                                                                       int32_t k0, int32_t K, int32_t koff ) {
    uint32_t const l_off = ( k0 + m_kl[J] < K ) ? m_off[J] + uint32_t( 4 * koff ) : kDmaOob;
    dma16( rsrc, l_off, lds_stage + ( wave * NJ + J ) * 1024 );
  }
};

// fragment readers of v_mfma_f32_32x32x2_f32: block i (32 rows), fragment
// step s (8 k): lane l feeds row l % 32, k = 8 s + 4 (l / 32) + e for the
// MFMA of k pair e = 0..3
template< int R, int BK, int NB, int MODE >
struct F32DmaFrag;

template< int R, int BK, int NB >
struct F32DmaFrag< R, BK, NB, LOAD_VEC_MN > {
  uint32_t m_addr[NB];   // byte address of (row, k = 4 (lane / 32)) in a stage

  __device__ inline void init( int row0, int lane ) {
    int const l_k = 4 * ( lane >> 5 );
#pragma unroll
    for( int l_i = 0; l_i < NB; l_i++ ) {
      int const l_r = row0 + 32 * l_i + ( lane & 31 );
      m_addr[l_i] = uint32_t( l_k * R * 4 ) + ( uint32_t( ( l_r >> 2 ) ^ int( swz_f32_mn( l_k ) ) ) << 4 )
                  + uint32_t( ( l_r & 3 ) * 4 );
    }
  }

  __device__ inline f32x4 read( char const * lds_stage, int i, int s ) const {
    float const * l_p = reinterpret_cast< float const * >( lds_stage + m_addr[i] + s * 8 * R * 4 );
    return f32x4{ l_p[0], l_p[R], l_p[2 * R], l_p[3 * R] };
  }
};

template< int R, int BK, int NB >
struct F32DmaFrag< R, BK, NB, LOAD_VEC_K > {
  uint32_t m_row_addr;
  uint32_t m_seg[BK / 8];

  __device__ inline void init( int row0, int lane ) {
    int const l_r = row0 + ( lane & 31 );
    m_row_addr = uint32_t( l_r * BK * 4 );
#pragma unroll
    for( int l_s = 0; l_s < BK / 8; l_s++ ) {
      m_seg[l_s] = uint32_t( ( 2 * l_s + ( lane >> 5 ) ) ^ int( swz_k( l_r ) ) ) << 4;
    }
  }

  __device__ inline f32x4 read( char const * lds_stage, int i, int s ) const {
    return *reinterpret_cast< f32x4 const * >( lds_stage + m_row_addr + m_seg[s] + i * 32 * BK * 4 );
  }
};

// KAFF false: K offsets from the plan's tables, which are staged in LDS
// (KTAB entries per operand, K <= KTAB) behind the stage buffers
template< int BM, int BN, int BK, int WM, int WN, int MA, int MB, bool KAFF >
__global__ __launch_bounds__( 64 * WM * WN, 1 )
void contract_f32_dma_kernel( ContractArgs a ) {
  constexpr int W   = WM * WN;
  constexpr int T   = 64 * W;
  constexpr int TM  = BM / WM / 32;
  constexpr int TN  = BN / WN / 32;
  constexpr int NS  = BK / 8;                  // fragment steps per k step
  constexpr int NMF = 4 * TM * TN;             // MFMAs per fragment step
  typedef F32DmaLoader< BM, BK, W, MA > LdA;
  typedef F32DmaLoader< BN, BK, W, MB > LdB;
  constexpr int SA  = LdA::STAGE_BYTES;
  constexpr int SB  = LdB::STAGE_BYTES;
  constexpr int ND  = LdA::NJ + LdB::NJ;       // DMA issues per wave and step
  constexpr int LDS_MAIN = 2 * ( SA + SB );
  constexpr int LDS_EPI  = EpilogueLds< BM, BN, WM, WN, TM, TN >::BYTES;
  constexpr int LDS_OPS   = LDS_MAIN > LDS_EPI ? LDS_MAIN : LDS_EPI;
  constexpr int KTAB      = kF32DmaMaxTableK;
  constexpr int LDS_BYTES = LDS_OPS + ( KAFF ? 0 : 2 * KTAB * 4 );
  static_assert( TM >= 1 && TN >= 1 && BK == 32, "fp32 DMA kernel: 32x32 MFMA blocks, k step 32" );
  static_assert( ND <= NMF, "at most one DMA issue per MFMA of the first fragment step" );

  __shared__ __attribute__( ( aligned( 1024 ) ) ) char l_lds[LDS_BYTES];

  // tile order as in the other contraction kernels: XCD-contiguous ranges,
  // groups of 8 tile rows
  int32_t const l_nblk = gridDim.x;
  int32_t l_bid = blockIdx.x;
  if( ( l_nblk & 7 ) == 0 ) l_bid = ( l_bid & 7 ) * ( l_nblk >> 3 ) + ( l_bid >> 3 );
  int32_t l_c, l_m0, l_n0;
  decode_tile< BM, BN >( a, l_bid, l_c, l_m0, l_n0 );

  int const l_lane = threadIdx.x & 63;
  int const l_wave = __builtin_amdgcn_readfirstlane( threadIdx.x >> 6 );
  int const l_wm   = l_wave / WN;
  int const l_wn   = l_wave - l_wm * WN;

  i32x4 const l_ra = make_rsrc( reinterpret_cast< float const * >( a.a ) + a.tc_a[l_c], kDmaOob );
  i32x4 const l_rb = make_rsrc( reinterpret_cast< float const * >( a.b ) + a.tc_b[l_c], kDmaOob );
  LdA l_lda;
  LdB l_ldb;
  int32_t * l_tka = reinterpret_cast< int32_t * >( l_lds + LDS_OPS );
  int32_t * l_tkb = l_tka + KTAB;
  if constexpr( KAFF ) {
    l_lda.init( a.tm_a, a.M, l_m0, a.sk_a, l_wave, l_lane );
    l_ldb.init( a.tn_b, a.N, l_n0, a.sk_b, l_wave, l_lane );
  }
  else {
    l_lda.init_tab( a.tm_a, a.M, l_m0, l_wave, l_lane );
    l_ldb.init_tab( a.tn_b, a.N, l_n0, l_wave, l_lane );
    // the K tables into LDS (K <= KTAB, planner); read before the first issue
    for( int32_t l_k = threadIdx.x; l_k < a.K; l_k += T ) {
      l_tka[l_k] = a.tk_a[l_k];
      l_tkb[l_k] = a.tk_b[l_k];
    }
    __syncthreads();
  }
  F32DmaFrag< BM, BK, TM, MA > l_fra;
  F32DmaFrag< BN, BK, TN, MB > l_frb;
  l_fra.init( l_wm * TM * 32, l_lane );
  l_frb.init( l_wn * TN * 32, l_lane );
  EpilogueTabs< BM, BN, T > l_tabs;
  l_tabs.load( a, l_m0, l_n0 );

  f32x16 l_acc[TM][TN];
#pragma unroll
  for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
    for( int l_j = 0; l_j < TN; l_j++ )
      l_acc[l_i][l_j] = f32x16( 0.0f );

  int32_t const  l_K    = a.K;
  int32_t const  l_nk   = ( l_K + BK - 1 ) / BK;
  uint32_t const l_kb_a = uint32_t( 4 * BK * a.sk_a );   // bytes per k step
  uint32_t const l_kb_b = uint32_t( 4 * BK * a.sk_b );
  uint32_t const l_lds0 = lds_addr( l_lds );

  // DMA issue d of a step: A chunks first, then B.  With a K table the
  // lane's k offsets are read from LDS first (l_koff, per issue).
  int32_t l_koff[ND];
  auto l_tab = [&]( int32_t l_k0 ) __attribute__( ( always_inline ) ) {
    if constexpr( !KAFF ) {
      static_for< ND >( [&]( auto dc ) __attribute__( ( always_inline ) ) {
        constexpr int l_d = decltype( dc )::value;
        if constexpr( l_d < LdA::NJ ) l_koff[l_d] = l_lda.template tab_entry< l_d >( l_tka, l_k0, l_K );
        else l_koff[l_d] = l_ldb.template tab_entry< l_d - LdA::NJ >( l_tkb, l_k0, l_K );
      } );
    }
  };
  auto l_issue = [&]( auto dc, uint32_t l_st, int32_t l_k0, uint32_t l_kt ) __attribute__( ( always_inline ) ) {
    constexpr int l_d = decltype( dc )::value;
    if constexpr( KAFF ) {
      if constexpr( l_d < LdA::NJ ) l_lda.template issue_one< l_d >( l_ra, l_st, l_wave, l_k0, l_K, l_kt * l_kb_a );
      else l_ldb.template issue_one< l_d - LdA::NJ >( l_rb, l_st + SA, l_wave, l_k0, l_K, l_kt * l_kb_b );
    }
    else {
      if constexpr( l_d < LdA::NJ ) l_lda.template issue_tab< l_d >( l_ra, l_st, l_wave, l_k0, l_K, l_koff[l_d] );
      else l_ldb.template issue_tab< l_d - LdA::NJ >( l_rb, l_st + SA, l_wave, l_k0, l_K, l_koff[l_d] );
    }
  };

  if( l_nk > 0 ) {
    l_tab( 0 );
    static_for< ND >( [&]( auto dc ) __attribute__( ( always_inline ) ) { l_issue( dc, l_lds0, 0, 0u ); } );
    wait_vmcnt< 0 >();
    barrier_lds();

    // one k step; TAIL (the last step only): skip the fragment steps wholly
    // past K, which hold zero padding (the first one always runs: it issues
    // the next step's loads).  The other steps are compiled without the test.
    auto l_step = [&]( int32_t l_kt, auto tail_c ) __attribute__( ( always_inline ) ) {
      constexpr bool TAIL = decltype( tail_c )::value;
      int const l_cur = l_kt & 1;
      char const * l_sa = l_lds + l_cur * ( SA + SB );
      char const * l_sb = l_sa + SA;
      // the other stage was last read in step kt - 1, which ended with a
      // barrier; the loads of the step past the last read zeros (k >= K) and
      // are drained by the wait below like all others
      uint32_t const l_nst = l_lds0 + uint32_t( l_cur ^ 1 ) * ( SA + SB );
      int32_t const  l_nk0 = ( l_kt + 1 ) * BK;
      int32_t const  l_kval = l_K - l_kt * BK;
      l_tab( l_nk0 );
      static_for< NS >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
        constexpr int l_s = decltype( sc )::value;
        if constexpr( TAIL && l_s > 0 ) {
          if( l_s * 8 >= l_kval ) return;
        }
        f32x4 l_fa[TM];
        f32x4 l_fb[TN];
#pragma unroll
        for( int l_i = 0; l_i < TM; l_i++ ) l_fa[l_i] = l_fra.read( l_sa, l_i, l_s );
#pragma unroll
        for( int l_j = 0; l_j < TN; l_j++ ) l_fb[l_j] = l_frb.read( l_sb, l_j, l_s );
        static_for< NMF >( [&]( auto fc ) __attribute__( ( always_inline ) ) {
          constexpr int l_f = decltype( fc )::value;
          // flat index f = (e, i, j), e the k pair inside the fragment
          constexpr int l_e = l_f / ( TM * TN );
          constexpr int l_i = ( l_f / TN ) % TM;
          constexpr int l_j = l_f % TN;
          l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x2f32( l_fa[l_i][l_e], l_fb[l_j][l_e],
                                                                  l_acc[l_i][l_j], 0, 0, 0 );
          if constexpr( l_s == 0 ) {
            // DMA issue d after MFMA (d + 1) * NMF / ND - 1 of the first fragment step
            static_for< ND >( [&]( auto dc ) __attribute__( ( always_inline ) ) {
              constexpr int l_d = decltype( dc )::value;
              if constexpr( ( l_d + 1 ) * NMF / ND - 1 == l_f ) l_issue( dc, l_nst, l_nk0, uint32_t( l_kt + 1 ) );
            } );
            __builtin_amdgcn_sched_barrier( 0 );
          }
        } );
      } );
      // the next stage has landed (own loads: vmcnt; everyone's: barrier) and
      // every wave is done reading this one
      wait_vmcnt< 0 >();
      wait_lgkmcnt0();
      barrier_lds();
    };
    for( int32_t l_kt = 0; l_kt + 1 < l_nk; l_kt++ ) l_step( l_kt, std::false_type() );
    l_step( l_nk - 1, std::true_type() );
  }

  epilogue< BM, BN, WM, WN, TM, TN, T >( a, l_acc, l_tabs, l_lds, l_c, l_m0, l_n0, l_wm, l_wn, l_lane );
}

}  // namespace kern

int launch_contract_f32_dma( int32_t ma, int32_t mb, ContractArgs const & a, uint32_t grid, hipStream_t stream ) {
  if( !a.k_affine && a.K > kern::kF32DmaMaxTableK ) {
    return fail( ETIR_COMPILATION_FAILED, "fp32 direct-to-LDS kernel: K table longer than its LDS copy" );
  }
  auto l_go = [&]( auto ma_c, auto mb_c ) {
    if( a.k_affine ) {
      hipLaunchKernelGGL( ( kern::contract_f32_dma_kernel< 128, 128, 32, 4, 2, decltype( ma_c )::value,
                                                           decltype( mb_c )::value, true > ),
                          dim3( grid ), dim3( 512 ), 0, stream, a );
    }
    else {
      hipLaunchKernelGGL( ( kern::contract_f32_dma_kernel< 128, 128, 32, 4, 2, decltype( ma_c )::value,
                                                           decltype( mb_c )::value, false > ),
                          dim3( grid ), dim3( 512 ), 0, stream, a );
    }
    return int( ETIR_SUCCESS );
  };
  typedef std::integral_constant< int32_t, LOAD_VEC_MN > Mn;
  typedef std::integral_constant< int32_t, LOAD_VEC_K >  Kc;
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_MN ) return l_go( Mn{}, Mn{} );
  if( ma == LOAD_VEC_MN && mb == LOAD_VEC_K )  return l_go( Mn{}, Kc{} );
  if( ma == LOAD_VEC_K  && mb == LOAD_VEC_MN ) return l_go( Kc{}, Mn{} );
  if( ma == LOAD_VEC_K  && mb == LOAD_VEC_K )  return l_go( Kc{}, Kc{} );
  return fail( ETIR_COMPILATION_FAILED, "no direct-to-LDS fp32 kernel for this load-mode combination" );
}

}  // namespace etir
