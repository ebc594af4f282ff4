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
// The global loads of step k+1 are issued between the MFMAs of the first
// fragment step of step k and their LDS stores between those of the last one
// (branch-free loaders, fixed by scheduling barriers).
#ifndef ETIR_CONTRACT_KERNEL_H
#define ETIR_CONTRACT_KERNEL_H

#include "etir_internal.h"
#include <type_traits>
#include <utility>

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
template<> struct InType< ETIR_FP64 > { typedef double   T; };

// Pitch (elements) of the [k][row] LDS layout.  bf16: 2*PK = 64 (mod 256) so
// the four k rows of one transpose read land in disjoint bank ranges; fp32:
// 4*PK = 32 (mod 64) so rows k and k+4 (the two lane groups) do not collide;
// fp64: 8*PK = 128 (mod 256) so the two k rows (16 lanes x 8 bytes each) read
// by one half-wave cover all 64 banks once.
template< int R, int ESZ >
struct KmPitch {
  static constexpr int bytes_raw = R * ESZ;
  static constexpr int pad = ( ESZ == 2 ) ? ( ( 64 - bytes_raw % 256 + 256 ) % 256 )
                           : ( ESZ == 8 ) ? ( ( 128 - bytes_raw % 256 + 256 ) % 256 )
                                          : ( ( 32 - bytes_raw % 64 + 64 ) % 64 );
  static constexpr int value = ( bytes_raw + pad ) / ESZ;
};

// compile-time loop: f( std::integral_constant< int, 0 .. N-1 > ); keeps
// register-array indices static where #pragma unroll alone may give up
template< typename F, int... Is >
__device__ __attribute__( ( always_inline ) ) inline void static_for_impl( F && f,
                                                                          std::integer_sequence< int, Is... > ) {
  ( f( std::integral_constant< int, Is >{} ), ... );
}
template< int N, typename F >
__device__ __attribute__( ( always_inline ) ) inline void static_for( F && f ) {
  static_for_impl( f, std::make_integer_sequence< int, N >{} );
}

// ---------------------------------------------------------------------------
// Operand loader: global -> registers -> LDS ([row][k], pitch LDK elements)
// ---------------------------------------------------------------------------
template< int R, int BK, int T, int ESZ, int MODE >
struct Loader;

// 16-byte vectors along K; the k index of a vector is fixed per thread.
//
// All vector loaders share one interface: init() once per tile, setup(k0)
// per K step (offsets and the validity mask), issue<I>() for the global load
// of vector I and put<I>() for its LDS store; load() and store() do all
// vectors at once.  Loads never branch: a vector outside the tensor (rows
// past M/N, k past K) reads row 0 / k 0 of the operand instead, which always
// exists, and put<I>() writes zeros for it.  Branch-free loads can be placed
// between MFMAs by the caller.
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_VEC_K > {
  static constexpr int V      = 16 / ESZ;           // elements per vector
  static constexpr int VPR    = BK / V;             // vectors per row
  static constexpr int COUNT  = R * VPR;
  static constexpr int NV     = ( COUNT + T - 1 ) / T;
  static constexpr int LDK    = BK + V;
  static_assert( NV <= 32, "validity mask" );

  u32x4    m_reg[NV];
  int32_t  m_row_off[NV];
  uint32_t m_row_ok;      // bit i: vector i is inside the tile and its row inside the tensor
  uint32_t m_ok;          // bit i: vector i of the current step holds data
  int32_t  m_koff;
  int      m_kv;

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
    m_kv = ( l_t % VPR ) * V;
    m_row_ok = 0;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      int const l_row = l_idx / VPR;
      int const l_g   = row0 + l_row;
      bool const l_ok = l_idx < COUNT && l_g < rows;
      if( l_ok ) m_row_ok |= 1u << l_i;
      m_row_off[l_i] = tab_rows[l_ok ? l_g : 0];
    }
  }

  template< bool KAFF >
  __device__ inline void setup( int32_t k0, int32_t K, int32_t const * tab_k, int32_t sk ) {
    int32_t const l_k  = k0 + m_kv;
    bool const    l_ok = l_k < K;
    int32_t const l_kc = l_ok ? l_k : 0;
    m_koff = KAFF ? l_kc * sk : tab_k[l_kc];
    m_ok   = l_ok ? m_row_ok : 0u;
  }

  template< int I, typename TE >
  __device__ inline void issue( TE const * base ) {
    m_reg[I] = *reinterpret_cast< u32x4 const * >( base + m_row_off[I] + m_koff );
  }

  template< int I, typename TE >
  __device__ inline void put( TE * lds ) {
    int const l_idx = int( threadIdx.x ) + I * T;
    if( COUNT % T == 0 || l_idx < COUNT ) {
      int const l_row = l_idx / VPR;
      u32x4 const l_v = ( ( m_ok >> I ) & 1u ) ? m_reg[I] : u32x4{ 0u, 0u, 0u, 0u };
      *reinterpret_cast< u32x4 * >( lds + l_row * LDK + m_kv ) = l_v;
    }
  }

  template< bool KAFF, typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t sk ) {
    setup< KAFF >( k0, K, tab_k, sk );
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { issue< decltype( ic )::value >( base ); } );
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { put< decltype( ic )::value >( lds ); } );
  }
};

// 8-byte vectors along K (fp32: two consecutive k), for K runs of even length
// that are not multiples of 4; LOAD_VEC_K's [row][k] LDS layout and pitch.
// Every K run has even length, so a vector is wholly inside K or past it.
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_VEC8_K > {
  static constexpr int V      = 8 / ESZ;            // elements per vector
  static constexpr int VPR    = BK / V;             // vectors per row
  static constexpr int COUNT  = R * VPR;
  static constexpr int NV     = ( COUNT + T - 1 ) / T;
  static constexpr int LDK    = BK + 16 / ESZ;
  static_assert( NV <= 32, "validity mask" );

  u32x2    m_reg[NV];
  int32_t  m_row_off[NV];
  uint32_t m_row_ok;
  uint32_t m_ok;
  int32_t  m_koff;
  int      m_kv;

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
    m_kv = ( l_t % VPR ) * V;
    m_row_ok = 0;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int const l_idx = l_t + l_i * T;
      int const l_row = l_idx / VPR;
      int const l_g   = row0 + l_row;
      bool const l_ok = l_idx < COUNT && l_g < rows;
      if( l_ok ) m_row_ok |= 1u << l_i;
      m_row_off[l_i] = tab_rows[l_ok ? l_g : 0];
    }
  }

  template< bool KAFF >
  __device__ inline void setup( int32_t k0, int32_t K, int32_t const * tab_k, int32_t sk ) {
    int32_t const l_k  = k0 + m_kv;
    bool const    l_ok = l_k < K;
    int32_t const l_kc = l_ok ? l_k : 0;
    m_koff = KAFF ? l_kc * sk : tab_k[l_kc];
    m_ok   = l_ok ? m_row_ok : 0u;
  }

  template< int I, typename TE >
  __device__ inline void issue( TE const * base ) {
    m_reg[I] = *reinterpret_cast< u32x2 const * >( base + m_row_off[I] + m_koff );
  }

  template< int I, typename TE >
  __device__ inline void put( TE * lds ) {
    int const l_idx = int( threadIdx.x ) + I * T;
    if( COUNT % T == 0 || l_idx < COUNT ) {
      int const l_row = l_idx / VPR;
      u32x2 const l_v = ( ( m_ok >> I ) & 1u ) ? m_reg[I] : u32x2{ 0u, 0u };
      *reinterpret_cast< u32x2 * >( lds + l_row * LDK + m_kv ) = l_v;
    }
  }

  template< bool KAFF, typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t sk ) {
    setup< KAFF >( k0, K, tab_k, sk );
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { issue< decltype( ic )::value >( base ); } );
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { put< decltype( ic )::value >( lds ); } );
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
  int32_t m_koff[V];
  bool    m_kok[V];
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

  // all table reads first, then all data reads: one wait for the tables
  template< bool KAFF >
  __device__ inline void setup( int32_t k0, int32_t K, int32_t const * tab_k, int32_t sk ) {
#pragma unroll
    for( int l_e = 0; l_e < V; l_e++ ) {
      int32_t const l_k = k0 + m_kv + l_e;
      m_kok[l_e] = l_k < K;
      m_koff[l_e] = 0;
      if( KAFF ) m_koff[l_e] = l_k * sk;
      else if( m_kok[l_e] ) m_koff[l_e] = tab_k[l_k];
    }
  }

  template< int I, typename TE >
  __device__ inline void issue( TE const * base ) {
    TE l_v[V];
#pragma unroll
    for( int l_e = 0; l_e < V; l_e++ ) {
      l_v[l_e] = TE( 0 );
      // row and k offsets each fit int32 (planner), their sum need not
      if( m_kok[l_e] && m_row_off[I] >= 0 ) l_v[l_e] = base[ int64_t( m_row_off[I] ) + m_koff[l_e] ];
    }
    m_reg[I] = *reinterpret_cast< u32x4 * >( l_v );
  }

  template< int I, typename TE >
  __device__ inline void put( TE * lds ) {
    int const l_idx = int( threadIdx.x ) + I * T;
    if( COUNT % T == 0 || l_idx < COUNT ) {
      int const l_row = l_idx / VPR;
      *reinterpret_cast< u32x4 * >( lds + l_row * LDK + m_kv ) = m_reg[I];
    }
  }

  template< bool KAFF, typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t sk ) {
    setup< KAFF >( k0, K, tab_k, sk );
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { issue< decltype( ic )::value >( base ); } );
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { put< decltype( ic )::value >( lds ); } );
  }
};

// 16-byte vectors of consecutive rows (unit stride along M or N) at one k,
// stored as loaded: LDS layout [k][row] with pitch PK elements.  The MFMA
// fragments (consecutive k for one row) are read back with the gfx950 LDS
// transpose read (bf16) or one 4-byte read per MFMA step (fp32), so no
// register transpose is needed and both the LDS writes (32 lanes cover one
// 512-byte row) and the reads are free of bank conflicts.
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_VEC_MN > {
  static constexpr int V      = 16 / ESZ;           // rows per vector
  static constexpr int VPK    = R / V;              // vectors per k row
  static constexpr int COUNT  = BK * VPK;
  static constexpr int NV     = COUNT / T;
  static constexpr int PK     = KmPitch< R, ESZ >::value;
  static_assert( COUNT % T == 0 && T % VPK == 0, "VEC_MN loader: tile/threads mismatch" );
  static_assert( NV <= 32, "validity mask" );

  u32x4    m_reg[NV];
  int32_t  m_koff[NV];
  int32_t  m_row_off;
  bool     m_row_ok;
  uint32_t m_ok;          // bit i: vector i of the current step holds data
  int      m_mv;
  int      m_k;

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
    m_mv = l_t % VPK;
    m_k  = l_t / VPK;
    int const l_g = row0 + m_mv * V;
    m_row_ok  = l_g < rows;
    m_row_off = tab_rows[m_row_ok ? l_g : 0];
  }

  template< bool KAFF >
  __device__ inline void setup( int32_t k0, int32_t K, int32_t const * tab_k, int32_t sk ) {
    m_ok = 0;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int32_t const l_k  = k0 + m_k + l_i * ( T / VPK );
      bool const    l_ok = l_k < K;
      int32_t const l_kc = l_ok ? l_k : 0;
      m_koff[l_i] = KAFF ? l_kc * sk : tab_k[l_kc];
      if( l_ok && m_row_ok ) m_ok |= 1u << l_i;
    }
  }

  template< int I, typename TE >
  __device__ inline void issue( TE const * base ) {
    m_reg[I] = *reinterpret_cast< u32x4 const * >( base + m_row_off + m_koff[I] );
  }

  template< int I, typename TE >
  __device__ inline void put( TE * lds ) {
    int const l_k = m_k + I * ( T / VPK );
    u32x4 const l_v = ( ( m_ok >> I ) & 1u ) ? m_reg[I] : u32x4{ 0u, 0u, 0u, 0u };
    *reinterpret_cast< u32x4 * >( lds + l_k * PK + m_mv * V ) = l_v;
  }

  template< bool KAFF, typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t sk ) {
    setup< KAFF >( k0, K, tab_k, sk );
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { issue< decltype( ic )::value >( base ); } );
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { put< decltype( ic )::value >( lds ); } );
  }
};

// 8-byte vectors of two consecutive rows (fp32), for row runs of even length
// that are not multiples of 4; LOAD_VEC_MN's [k][row] LDS layout and pitch.
// The operand's row count is even, so a vector is wholly inside or past it.
template< int R, int BK, int T, int ESZ >
struct Loader< R, BK, T, ESZ, LOAD_VEC8_MN > {
  static constexpr int V      = 8 / ESZ;            // rows per vector
  static constexpr int VPK    = R / V;              // vectors per k row
  static constexpr int COUNT  = BK * VPK;
  static constexpr int NV     = COUNT / T;
  static constexpr int PK     = KmPitch< R, ESZ >::value;
  static_assert( COUNT % T == 0 && T % VPK == 0, "VEC8_MN loader: tile/threads mismatch" );
  static_assert( NV <= 32, "validity mask" );

  u32x2    m_reg[NV];
  int32_t  m_koff[NV];
  int32_t  m_row_off;
  bool     m_row_ok;
  uint32_t m_ok;
  int      m_mv;
  int      m_k;

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0 ) {
    int const l_t = threadIdx.x;
    m_mv = l_t % VPK;
    m_k  = l_t / VPK;
    int const l_g = row0 + m_mv * V;
    m_row_ok  = l_g < rows;
    m_row_off = tab_rows[m_row_ok ? l_g : 0];
  }

  template< bool KAFF >
  __device__ inline void setup( int32_t k0, int32_t K, int32_t const * tab_k, int32_t sk ) {
    m_ok = 0;
#pragma unroll
    for( int l_i = 0; l_i < NV; l_i++ ) {
      int32_t const l_k  = k0 + m_k + l_i * ( T / VPK );
      bool const    l_ok = l_k < K;
      int32_t const l_kc = l_ok ? l_k : 0;
      m_koff[l_i] = KAFF ? l_kc * sk : tab_k[l_kc];
      if( l_ok && m_row_ok ) m_ok |= 1u << l_i;
    }
  }

  template< int I, typename TE >
  __device__ inline void issue( TE const * base ) {
    m_reg[I] = *reinterpret_cast< u32x2 const * >( base + m_row_off + m_koff[I] );
  }

  template< int I, typename TE >
  __device__ inline void put( TE * lds ) {
    int const l_k = m_k + I * ( T / VPK );
    u32x2 const l_v = ( ( m_ok >> I ) & 1u ) ? m_reg[I] : u32x2{ 0u, 0u };
    *reinterpret_cast< u32x2 * >( lds + l_k * PK + m_mv * V ) = l_v;
  }

  template< bool KAFF, typename TE >
  __device__ inline void load( TE const * base, int32_t k0, int32_t K,
                               int32_t const * tab_k, int32_t sk ) {
    setup< KAFF >( k0, K, tab_k, sk );
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { issue< decltype( ic )::value >( base ); } );
  }

  template< typename TE >
  __device__ inline void store( TE * lds ) {
    static_for< NV >( [&]( auto ic ) __attribute__( ( always_inline ) ) { put< decltype( ic )::value >( lds ); } );
  }
};

// ---------------------------------------------------------------------------
// MFMA fragment reads from LDS
//   fp32, v_mfma_f32_32x32x2_f32: step s (0..BK/2-1), lane group g = lane/32
//         feeds k = 8*(s/4) + 4*g + s%4
//   bf16, v_mfma_f32_32x32x16_bf16: step s (0..BK/16-1), lane group g feeds
//         k = 16*s + 8*g + (0..7)
// Both operands use the same assignment, so the sum over k is unchanged.
// ---------------------------------------------------------------------------
template< int ESZ, int MODE, int R, int BK >
struct Frag;

// [row][k] layout (LOAD_SCALAR, LOAD_VEC_K), fp32: one 16-byte read = 4 steps
template< int MODE, int R, int BK >
struct Frag< 4, MODE, R, BK > {
  static constexpr int LDK = BK + 4;
  __device__ static inline f32x4 read4( float const * lds, int row, int s4, int lane ) {
    return *reinterpret_cast< f32x4 const * >( lds + row * LDK + 8 * s4 + 4 * ( lane >> 5 ) );
  }
};

// [k][row] layout (LOAD_VEC_MN), fp32: one 4-byte read per step
template< int R, int BK >
struct Frag< 4, LOAD_VEC_MN, R, BK > {
  static constexpr int PK = KmPitch< R, 4 >::value;
  __device__ static inline f32x4 read4( float const * lds, int row, int s4, int lane ) {
    float const * l_p = lds + ( 8 * s4 + 4 * ( lane >> 5 ) ) * PK + row;
    return f32x4{ l_p[0], l_p[PK], l_p[2 * PK], l_p[3 * PK] };
  }
};

// [row][k] layout, bf16: one 16-byte read per step
template< int MODE, int R, int BK >
struct Frag< 2, MODE, R, BK > {
  static constexpr int LDK = BK + 8;
  __device__ static inline bf16x8 read8( uint16_t const * lds, int row, int s, int lane ) {
    return *reinterpret_cast< bf16x8 const * >( lds + row * LDK + 16 * s + 8 * ( lane >> 5 ) );
  }
};

// [k][row] layout, bf16: two transpose reads per step.  Within each group of
// 16 lanes, ds_read_b64_tr_b16 hands lane i element i%4 of the 8-byte chunks
// read by lanes 4j + i/4 (j = 0..3); lane L of the group therefore addresses
// row k = kb + L/4, columns 4*(L%4)..+3 of its 16-row slice, and receives the
// 4 consecutive k of row L.
template< int R, int BK >
struct Frag< 2, LOAD_VEC_MN, R, BK > {
  static constexpr int PK = KmPitch< R, 2 >::value;
  typedef short v4i16 __attribute__( ( ext_vector_type( 4 ) ) );
  typedef __attribute__( ( address_space( 3 ) ) ) v4i16 lds_v4i16;
  __device__ static inline bf16x8 read8( uint16_t const * lds, int row_base, int s, int lane ) {
    int const l_q   = lane >> 4;           // 16-lane group
    int const l_L   = lane & 15;
    int const l_row = row_base + 16 * ( l_q & 1 ) + 4 * ( l_L & 3 );
    int const l_kb  = 16 * s + 8 * ( l_q >> 1 ) + ( l_L >> 2 );
    uint16_t const * l_p0 = lds + l_kb * PK + l_row;
    uint16_t const * l_p1 = l_p0 + 4 * PK;
    v4i16 l_lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16( (lds_v4i16 *) ( l_p0 ) );
    v4i16 l_hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16( (lds_v4i16 *) ( l_p1 ) );
    typedef short v8i16 __attribute__( ( ext_vector_type( 8 ) ) );
    v8i16 l_all = __builtin_shufflevector( l_lo, l_hi, 0, 1, 2, 3, 4, 5, 6, 7 );
    return __builtin_bit_cast( bf16x8, l_all );
  }
};

template< int ESZ, int MODE, int R, int BK >
struct LdsSize {
  static constexpr int value = ( MODE == LOAD_VEC_MN ) ? BK * KmPitch< R, ESZ >::value
                                                       : R * ( BK + 16 / ESZ );
};

// ---------------------------------------------------------------------------
// epilogue: first/last-touch kernels and the output store of one tile.
// The tile's output (and aux) row/column offsets are staged in LDS first
// (s_tabs, 2*(BM+BN) int32): table reads from global memory between the
// stores would make every store wait for all earlier ones (one vector-memory
// counter on gfx9).  Accumulator layout of v_mfma_f32_32x32x*: register r of
// lane l holds row = 8*(r/4) + 4*(l/32) + r%4, column = l%32.
// ---------------------------------------------------------------------------
// a pointer whose value is the same in every lane, moved to scalar registers
// (buffer resources must be wave-uniform; the compiler cannot always prove it)
template< typename P >
__device__ __attribute__( ( always_inline ) ) inline P * uniform_ptr( P * p ) {
  uint64_t const l_v = reinterpret_cast< uint64_t >( p );
  uint32_t const l_lo = __builtin_amdgcn_readfirstlane( uint32_t( l_v ) );
  uint32_t const l_hi = __builtin_amdgcn_readfirstlane( uint32_t( l_v >> 32 ) );
  return reinterpret_cast< P * >( ( uint64_t( l_hi ) << 32 ) | l_lo );
}

// Epilogue of one tile: first/last-touch kernels and the output store.
//
// The tile's output (and aux) row/column offsets are staged in LDS first
// (2*(BM+BN) int32 at the start of `lds`): table reads from global memory
// between the stores would make every store wait for all earlier ones (one
// vector-memory counter on gfx9).  Accumulator layout of v_mfma_f32_32x32x*:
// register r of lane l holds row = 8*(r/4) + 4*(l/32) + r%4, column = l%32.
//
// Fast path -- fp32 output, first touch ZERO, last touch none or RELU,
// output byte offsets below 2^32: the four row offsets r%4 = 0..3 of one
// accumulator group come from one ds_read_b128, and every value is one
// non-temporal buffer_store_dword with a 32-bit byte offset from a per-tile
// base in scalar registers; full tiles store without bounds checks, edge
// tiles mask the stores of rows and columns past M and N.  When the output's
// column index is unit-stride each store writes two 128-byte runs (lanes
// 0-31 and 32-63).
//
// General path -- auxiliary tensors, accumulation into the output, bf16
// output: each wave stages one 32-row slab of its accumulators in
// its own LDS area and walks it in a rolled loop, consecutive lanes on
// consecutive columns.
template< int BM, int BN, int WM, int WN, int TM, int TN >
struct EpilogueLds {
  static constexpr int TABS  = 2 * ( BM + BN ) * 4;              // bytes of staged tables
  static constexpr int WCOLS = TN * 32;                          // columns of one wave
  static constexpr int PITCH = WCOLS + 4;                        // floats per slab row
  static constexpr int SLAB  = 32 * PITCH * 4;                   // bytes per wave
  static constexpr int BYTES = TABS + WM * WN * SLAB;
};

// cache policy of the output stores where every store instruction writes
// whole 128-byte runs: non-temporal (the output is written once and not read
// by the kernel; streaming it keeps the operand tiles that neighbouring
// workgroups still need in L2).  Where the columns are not unit-stride, the
// lines are completed by several stores or workgroups, and temporal stores
// let L2 merge them (eax,ebcdx->abcdx, the output's unit-stride dim x a C
// dim: 3.1 TFLOP/s with non-temporal stores).
constexpr int kStoreNt = 2;

// PARTIAL: an edge tile; only the first l_rows rows and l_cols columns of
// the tile (counted from the tile's origin) are stored
template< int TM, int TN, bool RELU, bool PARTIAL = false, bool NT = true >
__device__ __attribute__( ( always_inline ) ) inline void epilogue_fast_f32(
    float * l_base, f32x16 const ( &l_acc )[TM][TN], int32_t const * l_s_m_out,
    int32_t const * l_s_n_out, int l_row0, int l_col0, int l_lane, int l_rows = 0, int l_cols = 0 ) {
  int const l_lr = l_lane & 31;
  int const l_lg = l_lane >> 5;
  __amdgpu_buffer_rsrc_t const l_rs = __builtin_amdgcn_make_buffer_rsrc( uniform_ptr( l_base ), (short) 0,
                                                                         (int) 0xffffffff, 0x00020000 );
  uint32_t l_noff[TN];
  bool     l_nok[TN];
#pragma unroll
  for( int l_j = 0; l_j < TN; l_j++ ) {
    l_noff[l_j] = uint32_t( l_s_n_out[l_col0 + l_j * 32 + l_lr] ) * 4u;
    l_nok[l_j]  = !PARTIAL || ( l_col0 + l_j * 32 + l_lr < l_cols );
  }
  static_for< TM >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
    constexpr int l_i = decltype( ic )::value;
    static_for< 4 >( [&]( auto gc ) __attribute__( ( always_inline ) ) {
      constexpr int l_g = decltype( gc )::value;
      typedef int32_t i32x4v __attribute__( ( ext_vector_type( 4 ) ) );
      int const l_r0 = l_row0 + l_i * 32 + 8 * l_g + 4 * l_lg;
      i32x4v const l_m4 = *reinterpret_cast< i32x4v const * >( l_s_m_out + l_r0 );
      static_for< TN >( [&]( auto jc ) __attribute__( ( always_inline ) ) {
        constexpr int l_j = decltype( jc )::value;
        static_for< 4 >( [&]( auto ec ) __attribute__( ( always_inline ) ) {
          constexpr int l_e = decltype( ec )::value;
          float l_v = l_acc[l_i][l_j][4 * l_g + l_e];
          if constexpr( RELU ) l_v = fmaxf( l_v, 0.0f );
          if( !PARTIAL || ( l_nok[l_j] && l_r0 + l_e < l_rows ) ) {
            __builtin_amdgcn_raw_buffer_store_b32( __builtin_bit_cast( uint32_t, l_v ), l_rs,
                                                   uint32_t( l_m4[l_e] ) * 4u + l_noff[l_j], 0,
                                                   NT ? kStoreNt : 0 );
          }
        } );
      } );
    } );
  } );
}

// The epilogue's output/aux offsets of the tile rows and columns, loaded into
// registers when the workgroup starts (the loads complete under the main loop
// instead of adding a memory round trip after it) and staged in LDS at the
// epilogue.
template< int BM, int BN, int T >
struct EpilogueTabs {
  static constexpr int NM = ( BM + T - 1 ) / T;
  static constexpr int NN = ( BN + T - 1 ) / T;
  int32_t m_out[NM], m_aux[NM], n_out[NN], n_aux[NN];
  uint32_t m_valid;   // bit i: entry i of the m tables is a row inside M; bit 16 + i: n likewise

  // The loads read clamped indices unconditionally and nothing here uses
  // their values: a caller may issue them long before the tables are
  // staged without a wait for them (or for anything issued before them).
  __device__ inline void load( ContractArgs const & a, int32_t l_m0, int32_t l_n0 ) {
    static_assert( NM <= 16 && NN <= 16, "validity mask" );
    m_valid = 0;
#pragma unroll
    for( int l_i = 0; l_i < NM; l_i++ ) {
      int const l_x = threadIdx.x + l_i * T;
      int32_t const l_m = l_m0 + l_x;
      if( l_x < BM && l_m < a.M ) m_valid |= 1u << l_i;
      int32_t const l_mc = min( l_m, a.M - 1 );
      m_out[l_i] = a.tm_out[l_mc];
      m_aux[l_i] = a.tm_aux[l_mc];
    }
#pragma unroll
    for( int l_i = 0; l_i < NN; l_i++ ) {
      int const l_x = threadIdx.x + l_i * T;
      int32_t const l_n = l_n0 + l_x;
      if( l_x < BN && l_n < a.N ) m_valid |= 1u << ( 16 + l_i );
      int32_t const l_nc = min( l_n, a.N - 1 );
      n_out[l_i] = a.tn_out[l_nc];
      n_aux[l_i] = a.tn_aux[l_nc];
    }
  }

  // LDS layout: m_out[BM], m_aux[BM], n_out[BN], n_aux[BN]; entries outside
  // the tensor are 0
  __device__ inline void stage( int32_t * lds ) const {
#pragma unroll
    for( int l_i = 0; l_i < NM; l_i++ ) {
      int const l_x = threadIdx.x + l_i * T;
      if( l_x < BM ) {
        bool const l_ok = ( m_valid >> l_i ) & 1u;
        lds[l_x]      = l_ok ? m_out[l_i] : 0;
        lds[BM + l_x] = l_ok ? m_aux[l_i] : 0;
      }
    }
#pragma unroll
    for( int l_i = 0; l_i < NN; l_i++ ) {
      int const l_x = threadIdx.x + l_i * T;
      if( l_x < BN ) {
        bool const l_ok = ( m_valid >> ( 16 + l_i ) ) & 1u;
        lds[2 * BM + l_x]      = l_ok ? n_out[l_i] : 0;
        lds[2 * BM + BN + l_x] = l_ok ? n_aux[l_i] : 0;
      }
    }
  }
};

template< int BM, int BN, int WM, int WN, int TM, int TN, int T >
__device__ __attribute__( ( always_inline ) ) inline void epilogue( ContractArgs const & a,
                                                                    f32x16 const ( &l_acc )[TM][TN],
                                                                    EpilogueTabs< BM, BN, T > const & l_tabs,
                                                                    char * lds, int32_t l_c, int32_t l_m0,
                                                                    int32_t l_n0, int l_wm, int l_wn,
                                                                    int l_lane ) {
  typedef EpilogueLds< BM, BN, WM, WN, TM, TN > L;
  int32_t * l_s_m_out = reinterpret_cast< int32_t * >( lds );
  int32_t * l_s_m_aux = l_s_m_out + BM;
  int32_t * l_s_n_out = l_s_m_aux + BM;
  int32_t * l_s_n_aux = l_s_n_out + BN;
  bool const l_has_aux = ( a.aux != nullptr );
  l_tabs.stage( l_s_m_out );
  __syncthreads();

  int64_t const l_coff_out = a.tc_out[l_c];
  int const l_row0 = l_wm * TM * 32;      // first tile row of this wave
  int const l_col0 = l_wn * TN * 32;
  bool const l_full = ( l_m0 + BM <= a.M ) && ( l_n0 + BN <= a.N );
  if(    a.out_off32 && !a.out_bf16 && a.first_touch == ETIR_KTYPE_ZERO
      && ( a.last_touch == ETIR_KTYPE_UNDEFINED || a.last_touch == ETIR_KTYPE_RELU ) ) {
    // plain fp32 output: stores straight from the accumulators, edge tiles
    // with the rows and columns past M and N masked off (the staged table
    // entries of those are 0, never stored through)
    float * l_base = reinterpret_cast< float * >( a.out ) + l_coff_out;
    int const l_rows = int( min( int32_t( BM ), a.M - l_m0 ) );
    int const l_cols = int( min( int32_t( BN ), a.N - l_n0 ) );
    auto store = [&]( auto relu_c, auto partial_c, auto nt_c ) __attribute__( ( always_inline ) ) {
      epilogue_fast_f32< TM, TN, decltype( relu_c )::value, decltype( partial_c )::value, decltype( nt_c )::value >(
          l_base, l_acc, l_s_m_out, l_s_n_out, l_row0, l_col0, l_lane, l_rows, l_cols );
    };
    auto store_nt = [&]( auto relu_c, auto partial_c ) __attribute__( ( always_inline ) ) {
      if( a.out_nt ) store( relu_c, partial_c, std::true_type() );
      else           store( relu_c, partial_c, std::false_type() );
    };
    auto store_part = [&]( auto relu_c ) __attribute__( ( always_inline ) ) {
      if( l_full ) store_nt( relu_c, std::false_type() );
      else         store_nt( relu_c, std::true_type() );
    };
    if( a.last_touch == ETIR_KTYPE_RELU ) store_part( std::true_type() );
    else                                  store_part( std::false_type() );
    return;
  }

  int64_t const l_coff_aux = l_has_aux ? a.tc_aux[l_c] : 0;
  float const * l_aux_f = reinterpret_cast< float const * >( a.aux ) + l_coff_aux;
  uint16_t const * l_aux_h = reinterpret_cast< uint16_t const * >( a.aux ) + l_coff_aux;
  float * l_out_f = reinterpret_cast< float * >( a.out ) + l_coff_out;
  uint16_t * l_out_h = reinterpret_cast< uint16_t * >( a.out ) + l_coff_out;
  bool const l_read_out = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_UNDEFINED );
  bool const l_aux_first = ( a.first_touch == ETIR_KTYPE_ADD || a.first_touch == ETIR_KTYPE_COPY );
  bool const l_need_aux = l_has_aux && ( l_aux_first || a.last_touch == ETIR_KTYPE_ADD );
  int const l_lr = l_lane & 31;
  int const l_lg = l_lane >> 5;
  float * l_slab = reinterpret_cast< float * >( lds + L::TABS + ( l_wm * WN + l_wn ) * L::SLAB );

#pragma unroll
  for( int l_i = 0; l_i < TM; l_i++ ) {
    // stage slab i (32 rows x WCOLS) of this wave; the previous slab's reads
    // were issued earlier by this wave, and LDS executes one wave's accesses
    // in order
#pragma unroll
    for( int l_j = 0; l_j < TN; l_j++ )
#pragma unroll
      for( int l_r = 0; l_r < 16; l_r++ )
        l_slab[( 8 * ( l_r >> 2 ) + 4 * l_lg + ( l_r & 3 ) ) * L::PITCH + l_j * 32 + l_lr] = l_acc[l_i][l_j][l_r];
    for( int l_e = l_lane; l_e < 32 * L::WCOLS; l_e += 64 ) {
      int const l_row = l_e / L::WCOLS;
      int const l_col = l_e - l_row * L::WCOLS;
      int const l_ml = l_row0 + l_i * 32 + l_row;
      int const l_nl = l_col0 + l_col;
      if( l_m0 + l_ml >= a.M || l_n0 + l_nl >= a.N ) continue;
      int64_t const l_off = int64_t( l_s_n_out[l_nl] ) + l_s_m_out[l_ml];
      float l_v = l_slab[l_row * L::PITCH + l_col];
      float l_aux = 0.0f;
      if( l_need_aux ) {
        int64_t const l_aoff = int64_t( l_s_n_aux[l_nl] ) + l_s_m_aux[l_ml];
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

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
template< int DT, int BM, int BN, int BK, int WM, int WN, int MA, int MB, bool KAFF, int WPE >
__global__ __launch_bounds__( 64 * WM * WN, WPE )
void contract_kernel( ContractArgs a ) {
  typedef typename InType< DT >::T TE;
  constexpr int T    = 64 * WM * WN;
  constexpr int ESZ  = sizeof( TE );
  constexpr int TM   = BM / WM / 32;
  constexpr int TN   = BN / WN / 32;
  constexpr int LA   = lds_layout( MA );     // LDS layout of A and B
  constexpr int LB   = lds_layout( MB );
  constexpr int SZA  = LdsSize< ESZ, LA, BM, BK >::value;
  constexpr int SZB  = LdsSize< ESZ, LB, BN, BK >::value;
  static_assert( TM >= 1 && TN >= 1, "wave tile must hold at least one 32x32 block" );

  // one allocation: double-buffered A and B tiles, reused by the epilogue
  constexpr int LDS_MAIN  = 2 * ( SZA + SZB ) * ESZ;
  constexpr int LDS_EPI   = EpilogueLds< BM, BN, WM, WN, TM, TN >::BYTES;
  constexpr int LDS_BYTES = LDS_MAIN > LDS_EPI ? LDS_MAIN : LDS_EPI;
  static_assert( ( 2 * SZA * ESZ ) % 16 == 0, "B tile must stay 16-byte aligned" );
  __shared__ __attribute__( ( aligned( 16 ) ) ) char l_lds_raw[LDS_BYTES];
  TE ( *l_lds_a )[SZA] = reinterpret_cast< TE ( * )[SZA] >( l_lds_raw );
  TE ( *l_lds_b )[SZB] = reinterpret_cast< TE ( * )[SZB] >( l_lds_raw + 2 * SZA * ESZ );

  // XCD-aware order: consecutive workgroup ids are dispatched round-robin over
  // the 8 XCDs; remap so that each XCD works on one contiguous range of tiles
  // (sharing its L2), then walk tiles in groups of kGroupM tile rows.
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

  TE const * l_a = reinterpret_cast< TE const * >( a.a ) + a.tc_a[l_c];
  TE const * l_b = reinterpret_cast< TE const * >( a.b ) + a.tc_b[l_c];

  Loader< BM, BK, T, ESZ, MA > l_ld_a;
  Loader< BN, BK, T, ESZ, MB > l_ld_b;
  l_ld_a.init( a.tm_a, a.M, l_m0 );
  l_ld_b.init( a.tn_b, a.N, l_n0 );
  EpilogueTabs< BM, BN, T > l_tabs;
  l_tabs.load( a, l_m0, l_n0 );

  int const l_lane = threadIdx.x & 63;
  int const l_wave = threadIdx.x >> 6;
  int const l_wm   = l_wave / WN;
  int const l_wn   = l_wave - l_wm * WN;
  int const l_lr   = l_lane & 31;    // row (A) / column (B) inside a 32x32 block

  f32x16 l_acc[TM][TN];
#pragma unroll
  for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
    for( int l_j = 0; l_j < TN; l_j++ )
      l_acc[l_i][l_j] = f32x16( 0.0f );

  int32_t const l_nk = ( a.K + BK - 1 ) / BK;

  if( l_nk > 0 ) {
    l_ld_a.template load< KAFF >( l_a, 0, a.K, a.tk_a, a.sk_a );
    l_ld_b.template load< KAFF >( l_b, 0, a.K, a.tk_b, a.sk_b );
    l_ld_a.store( l_lds_a[0] );
    l_ld_b.store( l_lds_b[0] );
    __syncthreads();

    // rows of this wave's blocks; VEC_MN readers take the block base row
    int const l_ra = l_wm * TM * 32 + ( LA == LOAD_VEC_MN ? 0 : l_lr );
    int const l_rb = l_wn * TN * 32 + ( LB == LOAD_VEC_MN ? 0 : l_lr );

    // One K step on LDS buffer l_cur.  With MORE, the operand vectors of the
    // next step are loaded from global memory between the MFMAs of the first
    // fragment step and stored to the other buffer between those of the last
    // one, so that neither the load issue nor the LDS stores leave the MFMA
    // pipe idle.  The scheduling barriers keep that placement.  The last
    // step skips the fragment steps that lie wholly past K (l_kvalid valid k
    // in it): their LDS rows are zero padding.
    typedef Loader< BM, BK, T, ESZ, MA > LdA;
    typedef Loader< BN, BK, T, ESZ, MB > LdB;
    constexpr int NS  = ( DT == ETIR_FP32 ) ? BK / 8 : BK / 16;        // fragment steps
    constexpr int NMF = ( DT == ETIR_FP32 ) ? 4 * TM * TN : TM * TN;   // MFMAs per fragment step
    constexpr int NG  = NMF < 4 ? NMF : 4;                              // MFMA groups per fragment step
    constexpr int NL  = LdA::NV + LdB::NV;                              // vectors per thread and step
    constexpr int KF  = BK / NS;                                        // k per fragment step
    auto l_step = [&]( int l_cur, int32_t l_knext, int32_t l_kvalid, auto more_c ) __attribute__( ( always_inline ) ) {
      constexpr bool MORE = decltype( more_c )::value;
      TE const * l_sa = l_lds_a[l_cur];
      TE const * l_sb = l_lds_b[l_cur];
      TE * l_na = l_lds_a[l_cur ^ 1];
      TE * l_nb = l_lds_b[l_cur ^ 1];
      if constexpr( MORE ) {
        l_ld_a.template setup< KAFF >( l_knext, a.K, a.tk_a, a.sk_a );
        l_ld_b.template setup< KAFF >( l_knext, a.K, a.tk_b, a.sk_b );
      }
      static_for< NS >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
        constexpr int l_s = decltype( sc )::value;
        if constexpr( !MORE && l_s > 0 ) {
          if( l_s * KF >= l_kvalid ) return;
        }
        // fragments of step s: fp32 f32x4 (4 MFMA k-pairs), bf16 bf16x8 (one MFMA)
        typedef typename std::conditional< DT == ETIR_FP32, f32x4, bf16x8 >::type FragT;
        FragT l_fa[TM];
        FragT l_fb[TN];
#pragma unroll
        for( int l_i = 0; l_i < TM; l_i++ ) {
          if constexpr( DT == ETIR_FP32 )
            l_fa[l_i] = Frag< 4, LA, BM, BK >::read4( l_sa, l_ra + l_i * 32 + ( LA == LOAD_VEC_MN ? l_lr : 0 ),
                                                      l_s, l_lane );
          else
            l_fa[l_i] = Frag< 2, LA, BM, BK >::read8( l_sa, l_ra + l_i * 32, l_s, l_lane );
        }
#pragma unroll
        for( int l_j = 0; l_j < TN; l_j++ ) {
          if constexpr( DT == ETIR_FP32 )
            l_fb[l_j] = Frag< 4, LB, BN, BK >::read4( l_sb, l_rb + l_j * 32 + ( LB == LOAD_VEC_MN ? l_lr : 0 ),
                                                      l_s, l_lane );
          else
            l_fb[l_j] = Frag< 2, LB, BN, BK >::read8( l_sb, l_rb + l_j * 32, l_s, l_lane );
        }
        static_for< NG >( [&]( auto gc ) __attribute__( ( always_inline ) ) {
          constexpr int l_g = decltype( gc )::value;
          if constexpr( MORE && ( l_s == 0 || l_s == NS - 1 ) ) {
            static_for< NL >( [&]( auto vc ) __attribute__( ( always_inline ) ) {
              constexpr int l_v = decltype( vc )::value;
              // vector v goes to group v*NG/NL (NL >= NG) or group v (NL < NG)
              if constexpr( ( NL >= NG ? l_v * NG / NL : l_v ) == l_g ) {
                if constexpr( l_s == 0 ) {
                  if constexpr( l_v < LdA::NV ) l_ld_a.template issue< l_v >( l_a );
                  else                          l_ld_b.template issue< l_v - LdA::NV >( l_b );
                }
                if constexpr( l_s == NS - 1 ) {
                  if constexpr( l_v < LdA::NV ) l_ld_a.template put< l_v >( l_na );
                  else                          l_ld_b.template put< l_v - LdA::NV >( l_nb );
                }
              }
            } );
          }
          static_for< NMF / NG >( [&]( auto fc ) __attribute__( ( always_inline ) ) {
            constexpr int l_f = l_g * ( NMF / NG ) + decltype( fc )::value;
            if constexpr( DT == ETIR_FP32 ) {
              // flat index f = (e, i, j), e the k-pair inside the fragment
              constexpr int l_e = l_f / ( TM * TN );
              constexpr int l_i = ( l_f / TN ) % TM;
              constexpr int l_j = l_f % TN;
              l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x2f32( l_fa[l_i][l_e], l_fb[l_j][l_e],
                                                                      l_acc[l_i][l_j], 0, 0, 0 );
            }
            else {
              constexpr int l_i = l_f / TN;
              constexpr int l_j = l_f % TN;
              l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16( l_fa[l_i], l_fb[l_j],
                                                                         l_acc[l_i][l_j], 0, 0, 0 );
            }
          } );
          __builtin_amdgcn_sched_barrier( 0 );
        } );
      } );
    };

    int32_t l_kt = 0;
    for( ; l_kt + 1 < l_nk; l_kt++ ) {
      l_step( l_kt & 1, ( l_kt + 1 ) * BK, BK, std::true_type{} );
      __syncthreads();
    }
    l_step( l_kt & 1, 0, a.K - l_kt * BK, std::false_type{} );
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogue
  epilogue< BM, BN, WM, WN, TM, TN, T >( a, l_acc, l_tabs, l_lds_raw,
                                         l_c, l_m0, l_n0, l_wm, l_wn, l_lane );
}

}  // namespace kern
}  // namespace etir

#endif
