// gfx950 contraction kernel template.
//
// One launch computes a whole binary contraction
//   out[c][m][n] = touch( sum_k A[c][m][k] * B[c][n][k] )
// where c, m, n, k are FLATTENED indices over the fused C, M, N and K loops of
// the reference's loop IR (reference src/basic/constants.h:85-95) and every
// tensor address is  base + table_c[c] + table_m[m] + table_k[k]  (likewise
// for B and the output).  The tables are built by the planner from the loop
// strides; they make arbitrary strided layouts (non-adjacent M dims, many
// small modes) legal while the common case -- a unit-stride run along M/N or
// along K -- is detected by the planner and loaded with 16-byte (fp32) or
// 8/16-byte (bf16) vectors.
//
// What the reference does in its loop nest (ContractionBackend::contract_iter*,
// reference src/basic/binary/ContractionBackend.cpp:296-515) with first-touch
// kernels at the first K iteration and last-touch kernels at the last one
// (ContractionBackend.cpp:313-316, 495-515) is done here once per output
// element in the epilogue, because the whole K range is reduced inside one
// workgroup:
//   first touch ZERO  : v = sum
//   first touch COPY  : v = aux + sum                 (ContractionBackendTpp.cpp:136-140)
//   first touch ADD   : v = out + aux + sum           (ContractionBackendTpp.cpp:141-145)
//   first touch UNDEF : v = out + sum                 (accumulate into the output)
//   last touch  RELU  : v = max(v, 0)                 (ContractionBackendTpp.cpp:151-155)
//   last touch  ADD   : v = v + aux                   (ContractionBackendTpp.cpp:156-160)
//
// Structure: workgroup tile BM x BN, K step BK, WM x WN waves, each wave owns a
// (BM/WM) x (BN/WN) block of 32x32 MFMA tiles.  Operands are staged through a
// double-buffered LDS tile stored K-contiguous ([row][k], rows padded by 16 B
// so the 16-byte fragment reads of 8 consecutive lanes hit disjoint banks).
// Global loads for step k+1 are issued before the MFMAs of step k.
#ifndef ETIR_CONTRACT_KERNEL_H
#define ETIR_CONTRACT_KERNEL_H

#include "etir_internal.h"
#include <type_traits>

namespace etir {
namespace kern {

typedef float    f32x4  __attribute__( ( ext_vector_type( 4 ) ) );
typedef float    f32x16 __attribute__( ( ext_vector_type( 16 ) ) );
typedef __bf16   bf16x8 __attribute__( ( ext_vector_type( 8 ) ) );
typedef uint32_t u32x4  __attribute__( ( ext_vector_type( 4 ) ) );
typedef uint32_t u32x2  __attribute__( ( ext_vector_type( 2 ) ) );

__device__ inline float bf16_to_f32( uint16_t b ) {
  return __uint_as_float( uint32_t( b ) << 16 );
}

__device__ inline uint16_t f32_to_bf16_rne( float f ) {
  uint32_t u = __float_as_uint( f );
  if( ( u & 0x7f800000u ) == 0x7f800000u && ( u & 0x007fffffu ) ) {
    return uint16_t( ( u >> 16 ) | 0x40u );
  }
  u += 0x7fffu + ( ( u >> 16 ) & 1u );
  return uint16_t( u >> 16 );
}

// element storage type of the inputs: float or bf16 bits
template< int DT > struct InType;
template<> struct InType< ETIR_FP32 > { typedef float    T; };
template<> struct InType< ETIR_BF16 > { typedef uint16_t T; };

// ---------------------------------------------------------------------------
// Operand loader: global -> registers -> LDS ([row][k], pitch LDK elements)
// ---------------------------------------------------------------------------
template< int R, int BK, int T, int ESZ, int MODE >
struct Loader;

// 16-byte vectors along K; the k index of a vector is fixed per thread
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_VEC_K > {
  static constexpr int V      = 16 / ESZ;           // elements per vector
  static constexpr int VPR    = BK / V;             // vectors per row
  static constexpr int COUNT  = R * VPR;
  static constexpr int NV     = ( COUNT + T - 1 ) / T;
  static constexpr int LDK    = BK + V;

  u32x4   m_reg[NV];
  int32_t m_row_off[NV];
  int     m_kv;

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
    m_kv = ( l_t % VPR ) * V;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      int const l_row = l_idx / VPR;
      int const l_g   = row0 + l_row;
      m_row_off[l_i] = ( l_idx < COUNT && l_g < rows ) ? tab_rows[l_g] : -1;
    }
  }

  template< typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t k_affine, int32_t sk ) {
    int32_t const l_k = k0 + m_kv;
    bool const l_kok = l_k < K;
    int32_t l_koff = 0;
    if( l_kok ) l_koff = k_affine ? l_k * sk : tab_k[l_k];
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      if( l_kok && m_row_off[l_i] >= 0 ) {
        m_reg[l_i] = *reinterpret_cast< u32x4 const * >( base + m_row_off[l_i] + l_koff );
      }
      else {
        m_reg[l_i] = u32x4{ 0u, 0u, 0u, 0u };
      }
    }
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    int const l_t = threadIdx.x;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      if( COUNT % T == 0 || l_idx < COUNT ) {
        int const l_row = l_idx / VPR;
        *reinterpret_cast< u32x4 * >( lds + l_row * LDK + m_kv ) = m_reg[l_i];
      }
    }
  }
};

// element gathers through the tables; same thread layout as LOAD_VEC_K
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_SCALAR > {
  static constexpr int V      = 16 / ESZ;
  static constexpr int VPR    = BK / V;
  static constexpr int COUNT  = R * VPR;
  static constexpr int NV     = ( COUNT + T - 1 ) / T;
  static constexpr int LDK    = BK + V;

  u32x4   m_reg[NV];
  int32_t m_row_off[NV];
  int     m_kv;

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
    m_kv = ( l_t % VPR ) * V;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      int const l_row = l_idx / VPR;
      int const l_g   = row0 + l_row;
      m_row_off[l_i] = ( l_idx < COUNT && l_g < rows ) ? tab_rows[l_g] : -1;
    }
  }

  template< typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t k_affine, int32_t sk ) {
    int32_t l_koff[V];
    bool    l_kok[V];
#pragma unroll
    for( int l_e = 0; l_e < V; l_e++ ) {
      int32_t const l_k = k0 + m_kv + l_e;
      l_kok[l_e] = l_k < K;
      l_koff[l_e] = 0;
      if( l_kok[l_e] ) l_koff[l_e] = k_affine ? l_k * sk : tab_k[l_k];
    }
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      TE l_v[V];
#pragma unroll
      for( int l_e = 0; l_e < V; l_e++ ) {
        l_v[l_e] = TE( 0 );
        if( l_kok[l_e] && m_row_off[l_i] >= 0 ) l_v[l_e] = base[ m_row_off[l_i] + l_koff[l_e] ];
      }
      m_reg[l_i] = *reinterpret_cast< u32x4 * >( l_v );
    }
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    int const l_t = threadIdx.x;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      if( COUNT % T == 0 || l_idx < COUNT ) {
        int const l_row = l_idx / VPR;
        *reinterpret_cast< u32x4 * >( lds + l_row * LDK + m_kv ) = m_reg[l_i];
      }
    }
  }
};

// vectors of VR=4 consecutive rows (unit stride along M/N); each thread loads a
// VK x 4 micro-block (VK consecutive k) and transposes it in registers into
// 4 K-contiguous 16-byte LDS rows.
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_VEC_MN > {
  static constexpr int VR     = 4;                  // rows per global vector
  static constexpr int VK     = 16 / ESZ;           // k per LDS vector
  static constexpr int RG     = R / VR;             // row groups
  static constexpr int COUNT  = RG * ( BK / VK );
  static constexpr int NB     = ( COUNT + T - 1 ) / T;
  static constexpr int LDK    = BK + 16 / ESZ;
  // fp32: 16-byte row vectors, bf16: 8-byte row vectors
  typedef typename std::conditional< ESZ == 4, u32x4, u32x2 >::type RowVec;

  RowVec  m_reg[NB][VK];
  int32_t m_row_off[NB];
  int     m_rg[NB];
  int     m_kg[NB];

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
#pragma unroll
    for( int l_i = 0; l_i < NB; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      m_rg[l_i] = l_idx % RG;
      m_kg[l_i] = l_idx / RG;
      int const l_g = row0 + m_rg[l_i] * VR;
      m_row_off[l_i] = ( l_idx < COUNT && l_g < rows ) ? tab_rows[l_g] : -1;
    }
  }

  template< typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t k_affine, int32_t sk ) {
#pragma unroll
    for( int l_i = 0; l_i < NB; l_i++ ) {
      int32_t const l_kb = k0 + m_kg[l_i] * VK;
#pragma unroll
      for( int l_j = 0; l_j < VK; l_j++ ) {
        int32_t const l_k = l_kb + l_j;
        bool const l_ok = ( l_k < K ) && m_row_off[l_i] >= 0;
        if( l_ok ) {
          int32_t const l_koff = k_affine ? l_k * sk : tab_k[l_k];
          m_reg[l_i][l_j] = *reinterpret_cast< RowVec const * >( base + m_row_off[l_i] + l_koff );
        }
        else {
          m_reg[l_i][l_j] = RowVec( 0u );
        }
      }
    }
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
#pragma unroll
    for( int l_i = 0; l_i < NB; l_i++ ) {
      if( COUNT % T == 0 || ( int( threadIdx.x ) + l_i * T ) < COUNT ) {
        TE * l_dst = lds + ( m_rg[l_i] * VR ) * LDK + m_kg[l_i] * VK;
        if constexpr( ESZ == 4 ) {
          // 4x4 fp32 transpose: register renaming only
#pragma unroll
          for( int l_r = 0; l_r < 4; l_r++ ) {
            u32x4 l_w = u32x4{ m_reg[l_i][0][l_r], m_reg[l_i][1][l_r],
                               m_reg[l_i][2][l_r], m_reg[l_i][3][l_r] };
            *reinterpret_cast< u32x4 * >( l_dst + l_r * LDK ) = l_w;
          }
        }
        else {
          // 8(k) x 4(row) bf16 block: m_reg[k] = {row0|row1<<16, row2|row3<<16}
#pragma unroll
          for( int l_r = 0; l_r < 4; l_r++ ) {
            u32x4 l_w;
#pragma unroll
            for( int l_p = 0; l_p < 4; l_p++ ) {
              uint32_t const l_lo = m_reg[l_i][2 * l_p    ][l_r >> 1];
              uint32_t const l_hi = m_reg[l_i][2 * l_p + 1][l_r >> 1];
              l_w[l_p] = ( l_r & 1 ) ? ( ( l_lo >> 16 ) | ( l_hi & 0xffff0000u ) )
                                     : ( ( l_lo & 0xffffu ) | ( l_hi << 16 ) );
            }
            *reinterpret_cast< u32x4 * >( l_dst + l_r * LDK ) = l_w;
          }
        }
      }
    }
  }
};

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
template< int DT, int BM, int BN, int BK, int WM, int WN, int MA, int MB >
__global__ __launch_bounds__( 64 * WM * WN )
void contract_kernel( ContractArgs a ) {
  typedef typename InType< DT >::T TE;
  constexpr int T    = 64 * WM * WN;
  constexpr int ESZ  = sizeof( TE );
  constexpr int LDK  = BK + 16 / ESZ;
  constexpr int TM   = BM / WM / 32;
  constexpr int TN   = BN / WN / 32;
  static_assert( TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 block" );

  __shared__ __attribute__( ( aligned( 16 ) ) ) TE l_lds_a[2][BM * LDK];
  __shared__ __attribute__( ( aligned( 16 ) ) ) TE l_lds_b[2][BN * LDK];

  int32_t const l_ntiles = a.tiles_m * a.tiles_n;
  int32_t const l_bid    = blockIdx.x;
  int32_t const l_c      = l_bid / l_ntiles;
  int32_t const l_tile   = l_bid - l_c * l_ntiles;
  int32_t const l_tm     = l_tile / a.tiles_n;
  int32_t const l_tn     = l_tile - l_tm * a.tiles_n;
  int32_t const l_m0     = l_tm * BM;
  int32_t const l_n0     = l_tn * BN;

  TE const * l_a = reinterpret_cast< TE const * >( a.a ) + a.tc_a[l_c];
  TE const * l_b = reinterpret_cast< TE const * >( a.b ) + a.tc_b[l_c];

  Loader< BM, BK, T, ESZ, MA > l_ld_a;
  Loader< BN, BK, T, ESZ, MB > l_ld_b;
  l_ld_a.init( a.tm_a, a.M, l_m0 );
  l_ld_b.init( a.tn_b, a.N, l_n0 );

  int const l_lane = threadIdx.x & 63;
  int const l_wave = threadIdx.x >> 6;
  int const l_wm   = l_wave / WN;
  int const l_wn   = l_wave - l_wm * WN;
  int const l_lr   = l_lane & 31;    // row (A) / column (B) inside a 32x32 block
  int const l_lg   = l_lane >> 5;    // lane group: which k slice this lane feeds

  f32x16 l_acc[TM][TN];
#pragma unroll
  for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
    for( int l_j = 0; l_j < TN; l_j++ )
      l_acc[l_i][l_j] = f32x16( 0.0f );

  int32_t const l_nk = ( a.K + BK - 1 ) / BK;

  if( l_nk > 0 ) {
    l_ld_a.load( l_a, 0, a.K, a.tk_a, a.k_affine, a.sk_a );
    l_ld_b.load( l_b, 0, a.K, a.tk_b, a.k_affine, a.sk_b );
    l_ld_a.store( l_lds_a[0] );
    l_ld_b.store( l_lds_b[0] );
    __syncthreads();

    for( int32_t l_kt = 0; l_kt < l_nk; l_kt++ ) {
      int const l_cur = l_kt & 1;
      bool const l_more = ( l_kt + 1 ) < l_nk;
      if( l_more ) {
        l_ld_a.load( l_a, ( l_kt + 1 ) * BK, a.K, a.tk_a, a.k_affine, a.sk_a );
        l_ld_b.load( l_b, ( l_kt + 1 ) * BK, a.K, a.tk_b, a.k_affine, a.sk_b );
      }

      TE const * l_sa = l_lds_a[l_cur] + ( l_wm * TM * 32 + l_lr ) * LDK;
      TE const * l_sb = l_lds_b[l_cur] + ( l_wn * TN * 32 + l_lr ) * LDK;

      if constexpr( DT == ETIR_FP32 ) {
        // v_mfma_f32_32x32x2_f32: lane group g feeds k = g*BK/2 + s for step s
#pragma unroll
        for( int l_s4 = 0; l_s4 < BK / 8; l_s4++ ) {
          f32x4 l_fa[TM];
          f32x4 l_fb[TN];
#pragma unroll
          for( int l_i = 0; l_i < TM; l_i++ )
            l_fa[l_i] = *reinterpret_cast< f32x4 const * >( l_sa + l_i * 32 * LDK + l_lg * ( BK / 2 ) + 4 * l_s4 );
#pragma unroll
          for( int l_j = 0; l_j < TN; l_j++ )
            l_fb[l_j] = *reinterpret_cast< f32x4 const * >( l_sb + l_j * 32 * LDK + l_lg * ( BK / 2 ) + 4 * l_s4 );
#pragma unroll
          for( int l_e = 0; l_e < 4; l_e++ )
#pragma unroll
            for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
              for( int l_j = 0; l_j < TN; l_j++ )
                l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x2f32( l_fa[l_i][l_e], l_fb[l_j][l_e],
                                                                        l_acc[l_i][l_j], 0, 0, 0 );
        }
      }
      else {
        // v_mfma_f32_32x32x16_bf16: lane group g feeds k = 16*s + 8*g + (0..7)
#pragma unroll
        for( int l_s = 0; l_s < BK / 16; l_s++ ) {
          bf16x8 l_fa[TM];
          bf16x8 l_fb[TN];
#pragma unroll
          for( int l_i = 0; l_i < TM; l_i++ )
            l_fa[l_i] = *reinterpret_cast< bf16x8 const * >( l_sa + l_i * 32 * LDK + 16 * l_s + 8 * l_lg );
#pragma unroll
          for( int l_j = 0; l_j < TN; l_j++ )
            l_fb[l_j] = *reinterpret_cast< bf16x8 const * >( l_sb + l_j * 32 * LDK + 16 * l_s + 8 * l_lg );
#pragma unroll
          for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
            for( int l_j = 0; l_j < TN; l_j++ )
              l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16( l_fa[l_i], l_fb[l_j],
                                                                         l_acc[l_i][l_j], 0, 0, 0 );
        }
      }

      if( l_more ) {
        l_ld_a.store( l_lds_a[l_cur ^ 1] );
        l_ld_b.store( l_lds_b[l_cur ^ 1] );
      }
      __syncthreads();
    }
  }

  // ---------------------------------------------------------------- epilogue
  // 32x32 accumulator layout: register r of lane l holds
  //   row = 8*(r/4) + 4*(l/32) + r%4,  column = l%32
  int64_t const l_coff_out = a.tc_out[l_c];
  int64_t const l_coff_aux = ( a.aux != nullptr ) ? a.tc_aux[l_c] : 0;
  float const * l_aux_f = reinterpret_cast< float const * >( a.aux );
  uint16_t const * l_aux_h = reinterpret_cast< uint16_t const * >( a.aux );
  float * l_out_f = reinterpret_cast< float * >( a.out );
  uint16_t * l_out_h = reinterpret_cast< uint16_t * >( a.out );
  bool const l_read_out = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );

#pragma unroll
  for( int l_j = 0; l_j < TN; l_j++ ) {
    int32_t const l_n = l_n0 + ( l_wn * TN + l_j ) * 32 + l_lr;
    if( l_n >= a.N ) continue;
    int64_t const l_noff_out = l_coff_out + a.tn_out[l_n];
    int64_t const l_noff_aux = ( a.aux != nullptr ) ? l_coff_aux + a.tn_aux[l_n] : 0;
#pragma unroll
    for( int l_i = 0; l_i < TM; l_i++ ) {
#pragma unroll
      for( int l_r = 0; l_r < 16; l_r++ ) {
        int32_t const l_m = l_m0 + ( l_wm * TM + l_i ) * 32 + 8 * ( l_r >> 2 ) + 4 * l_lg + ( l_r & 3 );
        if( l_m >= a.M ) continue;
        int64_t const l_off = l_noff_out + a.tm_out[l_m];
        float l_v = l_acc[l_i][l_j][l_r];
        float l_aux = 0.0f;
        if( a.aux != nullptr && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD ) ) {
          int64_t const l_aoff = l_noff_aux + a.tm_aux[l_m];
          l_aux = a.out_bf16 ? bf16_to_f32( l_aux_h[l_aoff] ) : l_aux_f[l_aoff];
        }
        if( l_read_out ) {
          float const l_old = a.out_bf16 ? bf16_to_f32( l_out_h[l_off] ) : l_out_f[l_off];
          l_v = l_old + l_v;
        }
        if( l_aux_first ) l_v = l_aux + l_v;
        if( a.last_touch == ETIR_KTYPE_RELU ) l_v = fmaxf( l_v, 0.0f );
        else if( a.last_touch == ETIR_KTYPE_ADD ) l_v = l_v + l_aux;
        if( a.out_bf16 ) l_out_h[l_off] = f32_to_bf16_rne( l_v );
        else             l_out_f[l_off] = l_v;
      }
    }
  }
}

}  // namespace kern
}  // namespace etir

#endif
