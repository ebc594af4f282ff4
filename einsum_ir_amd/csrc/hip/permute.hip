// Permutation (unary COPY / ZERO / ADD) planner and gfx950 kernels.
//
// Behaviour follows the reference's unary path:
//   Unary::compile_base            reference src/backend/Unary.cpp:82-113
//     (sizes and input strides arrive in output-dimension order)
//   UnaryOptimizer / UnaryBackend  reference src/basic/unary/UnaryOptimizer.cpp:12-67,
//                                  src/basic/unary/UnaryBackend.cpp:59-226
//   UnaryBackendTpp kernels        reference src/basic/unary/UnaryBackendTpp.cpp:31-103
//     COPY -> identity / transpose, ZERO -> out = 0, ADD -> out = out + in.
//
// Device design (not a translation of the libxsmm 2-D TPP loop nest):
//   - size-1 dims are dropped and dims contiguous in both tensors are fused;
//   - if the unit-stride dim of the input (i) differs from the unit-stride dim
//     of the output (o) the (i, o) plane is moved through a 64x64 LDS tile:
//     coalesced 4-element vector reads along i, coalesced vector writes along
//     o, 65-element LDS rows so both the row-wise writes and the column-wise
//     reads hit 64 distinct banks; every other dim is a batch dim decoded once
//     per workgroup;
//   - if both of those unit-stride dims are shorter than a tile side, one of
//     them is at most 8 long or the input's is at most 16 long, the tile
//     instead covers the innermost contiguous run of each tensor (up to
//     two dims each, grown to at least 64 elements): reads run along the
//     input's run, writes along the output's, LDS reorders, and per-element
//     tile-relative offsets come from tables built once per plan (TILED);
//     the same holds when both tensors share one short unit-stride dim
//     (the tile then spans both tensors' next dims);
//   - if both innermost dims coincide otherwise the copy is vectorised along them;
//   - anything else is a one-thread-per-element gather.
#include "etir_internal.h"
#include <algorithm>
#include <cinttypes>
#include <cstdio>
#include <limits>
#include <numeric>
#include <sstream>

namespace etir {

namespace {

struct bf16_t { uint16_t bits; };

template< typename T > struct Elem;
template<> struct Elem< float > {
  typedef float storage;
  __device__ static inline float add( float a, float b ) { return a + b; }
};
template<> struct Elem< double > {
  typedef double storage;
  __device__ static inline double add( double a, double b ) { return a + b; }
};
template<> struct Elem< uint16_t > {  // bf16 bits
  typedef uint16_t storage;
  __device__ static inline uint16_t add( uint16_t a, uint16_t b ) {
    float fa = __uint_as_float( uint32_t( a ) << 16 );
    float fb = __uint_as_float( uint32_t( b ) << 16 );
    float s  = fa + fb;
    uint32_t u = __float_as_uint( s );
    // round to nearest even; NaN stays NaN
    if( ( u & 0x7f800000u ) == 0x7f800000u && ( u & 0x007fffffu ) ) {
      return uint16_t( ( u >> 16 ) | 0x40u );
    }
    u += 0x7fffu + ( ( u >> 16 ) & 1u );
    return uint16_t( u >> 16 );
  }
};

template< typename T >
struct alignas( 4 * sizeof( T ) ) Vec4 { T v[4]; };

// N consecutive elements moved as one vector
template< typename T, int N >
struct alignas( N * sizeof( T ) ) VecN { T v[N]; };


constexpr int kTile = 64;
constexpr int kThreads = 256;

// REG4 takes permutations whose shorter unit-stride dim is at most this long
// (kReg4MaxShort elements of 4 bytes), and those whose two
// unit-stride dims are at most 32 long and whole 128-byte lines each (fp32
// 32 x 32: 74 % of HBM peak against 58 % tiled; 24 x 32, whose 96-byte input
// runs split lines: 47 % against 53 % tiled)
constexpr int64_t kReg4MaxShort = 16;
constexpr int kPermTileMax = 4096;   // elements of a TILED tile

// 16-byte store that does not keep the line in the caches (the output is
// written once and not read again by the kernel)
template< typename V >
__device__ inline void store_stream( V * p, V const & v ) {
  if constexpr( sizeof( V ) == 16 ) {
    typedef uint32_t u4 __attribute__( ( ext_vector_type( 4 ) ) );
    __builtin_nontemporal_store( __builtin_bit_cast( u4, v ), reinterpret_cast< u4 * >( p ) );
  }
  else {
    *p = v;
  }
}

// Next digit of a workgroup index in the mixed radix of the grid: returns
// io_rest % i_size and leaves io_rest / i_size.  Every radix is a factor of
// the grid size, which the launch keeps below 2^31, so 32-bit unsigned
// division is exact; the 64-bit one is a long emulated sequence that delayed
// every workgroup's first load by several hundred instructions.
__device__ inline int64_t grid_digit( uint32_t & io_rest, int64_t i_size ) {
  uint32_t const l_s = uint32_t( i_size );
  uint32_t const l_q = io_rest / l_s;
  uint32_t const l_r = io_rest - l_q * l_s;
  io_rest = l_q;
  return int64_t( l_r );
}

// LDS-tiled transpose of one TI x TO (i, o) tile per workgroup (64 x 64, or
// 128 x 32 / 32 x 128 when one unit-stride dim is at most 32 long and the
// other at least 128: a 64 x 64 tile would be half empty).  Threads move 4
// consecutive elements: reads run along i (TI / 4 threads per o row), writes
// along o (TO / 4 threads per i row), four passes each.  The LDS pitch is
// TI + 1 for square tiles and TI + 2 otherwise, which spreads the write
// phase's column reads over distinct banks.
// The transpose for 2-byte elements with 16-byte reads: a TI x TO tile
// (TI = 128 along the input's unit-stride dim i) read as 8 elements per
// vector, written as 4 per vector along the output's unit-stride dim o
// (output runs may be as short as 4 elements).  With 8-byte reads the same
// moves ran at 41-51 % of HBM peak (bf16 abcd->bdac 36,48,36,512: 41 -> 51 %;
// 72,96,72,1024 on TO = 32: 42 -> 54 %; abcd->dbca 128^4, beyond the
// Infinity Cache: 51 -> 59 %).  LDS rows are padded by 4 bytes so that the
// column reads of the write phase step one bank per row.  VEC false (no
// vector alignment, a.vec_ok 0): every access is one element (a separate
// instantiation: the run-time choice inside one kernel cost 10 %).
// FOLD: o is the output's unit-stride dim and the one after it together
// (a.o1_size > 0), contiguous in the output, two strides in the input, so an
// output dim that is not a multiple of the tile still fills it (bf16
// abcd->bdac 36,48,36,512: o runs over c and a, 1296 elements, instead of
// 36 of every 64).
template< typename T, int TI, int TO, bool VEC, bool FOLD >
__global__ __launch_bounds__( kThreads )
void perm_transpose16_kernel( PermArgs a ) {
  static_assert( sizeof( T ) == 2, "16-byte reads of 8 elements" );
  constexpr int VR = 8;
  constexpr int VW = 4;
  constexpr int PITCH = TI + 2;
  constexpr int RT = TI / VR;             // read: threads per o row
  constexpr int WT = TO / VW;             // write: threads per i row
  constexpr int RP = TI * TO / ( VR * kThreads );
  constexpr int WP = TI * TO / ( VW * kThreads );
  static_assert( RP * VR * kThreads == TI * TO && WP * VW * kThreads == TI * TO, "whole passes" );
  __shared__ T l_tile[TO][PITCH];

  uint32_t l_bid = blockIdx.x;
  int64_t const l_ti = grid_digit( l_bid, a.tiles_i );
  int64_t const l_to = grid_digit( l_bid, a.tiles_o );
  int64_t l_off_in  = 0;
  int64_t l_off_out = 0;
  for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
    int64_t const l_idx = grid_digit( l_bid, a.batch_size[l_d] );
    l_off_in  += l_idx * a.batch_s_in[l_d];
    l_off_out += l_idx * a.batch_s_out[l_d];
  }
  T const * l_in  = reinterpret_cast< T const * >( a.in )  + l_off_in;
  T       * l_out = reinterpret_cast< T       * >( a.out ) + l_off_out;
  int64_t const l_i0 = l_ti * TI;
  int64_t const l_o0 = l_to * TO;
  int const l_t = threadIdx.x;

  // read: rows along o, VR consecutive i per thread (all loads of the
  // thread in flight before the first LDS store)
  int const l_c = l_t % RT;
  int const l_r = l_t / RT;
  VecN< T, VR > l_v[RP];
#pragma unroll
  for( int l_p = 0; l_p < RP; l_p++ ) {
    int64_t const l_o = l_o0 + l_r + ( kThreads / RT ) * l_p;
    int64_t const l_i = l_i0 + VR * l_c;
    int64_t l_row;                          // input offset of row o
    if constexpr( FOLD ) {
      uint32_t const l_o2 = __umulhi( uint32_t( l_o ), a.o1_magic );
      uint32_t const l_o1 = uint32_t( l_o ) - l_o2 * uint32_t( a.o1_size );
      l_row = int64_t( l_o1 ) * a.s_in_o + int64_t( l_o2 ) * a.s_in_o2;
    }
    else {
      l_row = l_o * a.s_in_o;
    }
#pragma unroll
    for( int l_e = 0; l_e < VR; l_e++ ) l_v[l_p].v[l_e] = T( 0 );
    if constexpr( VEC ) {
      if( l_o < a.size_o && l_i < a.size_i ) {
        l_v[l_p] = *reinterpret_cast< VecN< T, VR > const * >( l_in + l_row + l_i );
      }
    }
    else {
#pragma unroll
      for( int l_e = 0; l_e < VR; l_e++ ) {
        if( l_o < a.size_o && l_i + l_e < a.size_i ) l_v[l_p].v[l_e] = l_in[l_row + l_i + l_e];
      }
    }
  }
#pragma unroll
  for( int l_p = 0; l_p < RP; l_p++ ) {
    int const l_row = l_r + ( kThreads / RT ) * l_p;
#pragma unroll
    for( int l_e = 0; l_e < VR; l_e++ ) l_tile[l_row][VR * l_c + l_e] = l_v[l_p].v[l_e];
  }

  __syncthreads();

  // write: rows along i, VW consecutive o per thread
  int const l_wc = l_t % WT;
  int const l_wr = l_t / WT;
#pragma unroll
  for( int l_p = 0; l_p < WP; l_p++ ) {
    int const l_row = l_wr + ( kThreads / WT ) * l_p;
    int64_t const l_i = l_i0 + l_row;
    int64_t const l_o = l_o0 + VW * l_wc;
    VecN< T, VW > l_w;
#pragma unroll
    for( int l_e = 0; l_e < VW; l_e++ ) l_w.v[l_e] = l_tile[VW * l_wc + l_e][l_row];
    if constexpr( VEC ) {
      if( l_i < a.size_i && l_o < a.size_o ) {
        VecN< T, VW > * l_ptr = reinterpret_cast< VecN< T, VW > * >( l_out + l_i * a.s_out_i + l_o );
        if( a.add ) {
          VecN< T, VW > const l_old = *l_ptr;
#pragma unroll
          for( int l_e = 0; l_e < VW; l_e++ ) l_w.v[l_e] = Elem< T >::add( l_old.v[l_e], l_w.v[l_e] );
        }
        *l_ptr = l_w;
      }
    }
    else {
#pragma unroll
      for( int l_e = 0; l_e < VW; l_e++ ) {
        if( l_i < a.size_i && l_o + l_e < a.size_o ) {
          T * l_ptr = l_out + l_i * a.s_out_i + l_o + l_e;
          *l_ptr = a.add ? Elem< T >::add( *l_ptr, l_w.v[l_e] ) : l_w.v[l_e];
        }
      }
    }
  }
}

template< typename T, int TI, int TO >
__global__ __launch_bounds__( kThreads )
void perm_transpose_kernel( PermArgs a ) {
  static_assert( TI * TO == 4 * 4 * kThreads, "four passes of 4 elements per thread" );
  constexpr int PITCH = TI + ( TI == TO ? 1 : 2 );
  constexpr int RT = TI / 4;              // read: threads per o row
  constexpr int WT = TO / 4;              // write: threads per i row
  __shared__ T l_tile[TO][PITCH];

  uint32_t l_bid = blockIdx.x;
  int64_t const l_ti = grid_digit( l_bid, a.tiles_i );
  int64_t const l_to = grid_digit( l_bid, a.tiles_o );

  int64_t l_off_in  = 0;
  int64_t l_off_out = 0;
  for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
    int64_t const l_idx = grid_digit( l_bid, a.batch_size[l_d] );
    l_off_in  += l_idx * a.batch_s_in[l_d];
    l_off_out += l_idx * a.batch_s_out[l_d];
  }

  T const * l_in  = reinterpret_cast< T const * >( a.in )  + l_off_in;
  T       * l_out = reinterpret_cast< T       * >( a.out ) + l_off_out;

  int64_t const l_i0 = l_ti * TI;
  int64_t const l_o0 = l_to * TO;
  int const l_t  = threadIdx.x;
  int const l_c4 = l_t % RT;
  int const l_r  = l_t / RT;

  // read: rows along o, 4 consecutive i per thread
#pragma unroll
  for( int l_p = 0; l_p < 4; l_p++ ) {
    int const l_row = l_r + ( kThreads / RT ) * l_p;
    int64_t const l_o = l_o0 + l_row;
    int64_t const l_i = l_i0 + 4 * l_c4;
    T l_v[4] = { T(0), T(0), T(0), T(0) };
    if( a.vec_ok ) {
      if( l_o < a.size_o && l_i < a.size_i ) {
        Vec4< T > l_tmp = *reinterpret_cast< Vec4< T > const * >( l_in + l_o * a.s_in_o + l_i );
#pragma unroll
        for( int l_e = 0; l_e < 4; l_e++ ) l_v[l_e] = l_tmp.v[l_e];
      }
    }
    else {
#pragma unroll
      for( int l_e = 0; l_e < 4; l_e++ ) {
        if( l_o < a.size_o && l_i + l_e < a.size_i ) {
          l_v[l_e] = l_in[ l_o * a.s_in_o + l_i + l_e ];
        }
      }
    }
#pragma unroll
    for( int l_e = 0; l_e < 4; l_e++ ) l_tile[l_row][4 * l_c4 + l_e] = l_v[l_e];
  }

  __syncthreads();

  // write: rows along i, 4 consecutive o per thread
  int const l_wc4 = l_t % WT;
  int const l_wr  = l_t / WT;
#pragma unroll
  for( int l_p = 0; l_p < 4; l_p++ ) {
    int const l_row = l_wr + ( kThreads / WT ) * l_p;
    int64_t const l_i = l_i0 + l_row;
    int64_t const l_o = l_o0 + 4 * l_wc4;
    T l_v[4];
#pragma unroll
    for( int l_e = 0; l_e < 4; l_e++ ) l_v[l_e] = l_tile[4 * l_wc4 + l_e][l_row];

    if( a.vec_ok ) {
      if( l_i < a.size_i && l_o < a.size_o ) {
        Vec4< T > * l_ptr = reinterpret_cast< Vec4< T > * >( l_out + l_i * a.s_out_i + l_o );
        if( a.add ) {
          Vec4< T > l_old = *l_ptr;
#pragma unroll
          for( int l_e = 0; l_e < 4; l_e++ ) l_v[l_e] = Elem< T >::add( l_old.v[l_e], l_v[l_e] );
        }
        Vec4< T > l_tmp;
#pragma unroll
        for( int l_e = 0; l_e < 4; l_e++ ) l_tmp.v[l_e] = l_v[l_e];
        if( a.nt_store ) store_stream( l_ptr, l_tmp );
        else             *l_ptr = l_tmp;
      }
    }
    else {
#pragma unroll
      for( int l_e = 0; l_e < 4; l_e++ ) {
        if( l_i < a.size_i && l_o + l_e < a.size_o ) {
          T * l_ptr = l_out + l_i * a.s_out_i + l_o + l_e;
          *l_ptr = a.add ? Elem< T >::add( *l_ptr, l_v[l_e] ) : l_v[l_e];
        }
      }
    }
  }
}

// One tile per workgroup over the union of the input's and the output's
// innermost contiguous runs (up to kPermTileDims dims); other dims are batch
// dims.  Reads follow tab_r (input order, consecutive threads on consecutive
// input addresses), writes follow tab_w (output order); edge tiles skip the
// elements whose coordinates reach past a tile dim's size.
__device__ inline bool perm_tile_inside( uint32_t coords, uint32_t lim, int nd ) {
  for( int l_k = 0; l_k < nd; l_k++ ) {
    if( ( ( coords >> ( 8 * l_k ) ) & 255u ) >= ( ( lim >> ( 8 * l_k ) ) & 255u ) ) return false;
  }
  return true;
}

template< typename T, int V >
__global__ __launch_bounds__( kThreads )
void perm_tiled_kernel( PermArgs a ) {
  extern __shared__ __attribute__( ( aligned( 16 ) ) ) char l_lds_raw[];
  T * l_tile = reinterpret_cast< T * >( l_lds_raw );

  uint32_t l_bid = blockIdx.x;
  int64_t l_off_in = 0, l_off_out = 0;
  uint32_t l_lim = 0;
  bool l_full = true;
  for( int l_k = 0; l_k < a.tile_nd; l_k++ ) {
    int64_t const l_b = grid_digit( l_bid, a.tile_nblk[l_k] );
    int64_t const l_c0 = l_b * a.tile_ext[l_k];
    int64_t const l_left = a.tile_size[l_k] - l_c0;
    int64_t const l_n = l_left < a.tile_ext[l_k] ? l_left : a.tile_ext[l_k];
    l_full = l_full && ( l_n == a.tile_ext[l_k] );
    l_lim |= uint32_t( l_n ) << ( 8 * l_k );
    l_off_in  += l_c0 * a.tile_s_in[l_k];
    l_off_out += l_c0 * a.tile_s_out[l_k];
  }
  for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
    int64_t const l_idx = grid_digit( l_bid, a.batch_size[l_d] );
    l_off_in  += l_idx * a.batch_s_in[l_d];
    l_off_out += l_idx * a.batch_s_out[l_d];
  }
  T const * l_in  = reinterpret_cast< T const * >( a.in ) + l_off_in;
  T       * l_out = reinterpret_cast< T * >( a.out ) + l_off_out;
  // V consecutive elements of an entry share every coordinate but the
  // innermost run dim's, whose size is a multiple of V: they are all inside
  // a tile dim's size or all outside
  int const l_nv = a.tile_n / V;
  bool const l_vec = ( V > 1 ) && a.vec_ok;

  // read: entry j = input-order elements V j .. V j + V - 1, contiguous in the input
  for( int l_j = threadIdx.x; l_j < l_nv; l_j += kThreads ) {
    if( !( l_full || perm_tile_inside( uint32_t( a.tab_rc[l_j] ), l_lim, a.tile_nd ) ) ) continue;
    int32_t const l_off = a.tab_r[l_j];
    T l_v[V];
    if( l_vec ) {
      Vec4< T > const l_x = *reinterpret_cast< Vec4< T > const * >( l_in + l_off );
#pragma unroll
      for( int l_q = 0; l_q < V; l_q++ ) l_v[l_q] = l_x.v[l_q];
    }
    else {
#pragma unroll
      for( int l_q = 0; l_q < V; l_q++ ) l_v[l_q] = l_in[l_off + l_q];
    }
    int const l_t = V * l_j;
#pragma unroll
    for( int l_q = 0; l_q < V; l_q++ ) l_tile[l_t + l_q + ( ( l_t + l_q ) >> 6 ) * a.tile_pad] = l_v[l_q];
  }
  __syncthreads();
  // write: entry j = output-order elements V j .. V j + V - 1, contiguous in
  // the output; {output offset, input-order index of the first element}: the
  // others follow at tile_t_step (they differ only in the output's
  // unit-stride dim)
  int2 const * l_tw = reinterpret_cast< int2 const * >( a.tab_w );
  for( int l_j = threadIdx.x; l_j < l_nv; l_j += kThreads ) {
    if( !( l_full || perm_tile_inside( uint32_t( a.tab_wc[l_j] ), l_lim, a.tile_nd ) ) ) continue;
    int2 const l_e = l_tw[l_j];
    T l_v[V];
#pragma unroll
    for( int l_q = 0; l_q < V; l_q++ ) {
      int const l_t = l_e.y + l_q * a.tile_t_step;
      l_v[l_q] = l_tile[l_t + ( l_t >> 6 ) * a.tile_pad];
    }
    T * l_ptr = l_out + l_e.x;
    if( l_vec ) {
      Vec4< T > l_x;
      if( a.add ) {
        Vec4< T > const l_old = *reinterpret_cast< Vec4< T > const * >( l_ptr );
#pragma unroll
        for( int l_q = 0; l_q < V; l_q++ ) l_x.v[l_q] = Elem< T >::add( l_old.v[l_q], l_v[l_q] );
      }
      else {
#pragma unroll
        for( int l_q = 0; l_q < V; l_q++ ) l_x.v[l_q] = l_v[l_q];
      }
      *reinterpret_cast< Vec4< T > * >( l_ptr ) = l_x;
    }
    else {
#pragma unroll
      for( int l_q = 0; l_q < V; l_q++ ) {
        l_ptr[l_q] = a.add ? Elem< T >::add( l_ptr[l_q], l_v[l_q] ) : l_v[l_q];
      }
    }
  }
}

// Short unit-stride dims (REG4): 4 x 4 blocks transposed in registers, whole
// 16-byte rows exchanged through LDS.  i is the input's unit-stride dim, o
// the output's, c the dim walked next (the one that continues the input's
// run, or the output's); a workgroup takes all of i and o and c_chunk values
// of c (size_i * size_o * c_chunk <= 4096 elements).
//   read:  thread (ig, c, og) -- ig fastest -- loads the four 16-byte rows
//          in[o = 4 og + r][c][i = 4 ig .. 4 ig + 3], r = 0..3: one load
//          instruction of a wave covers one input row o over a contiguous
//          run of (c, i);
//   swap:  the 4 x 4 block is transposed by renaming registers, and its four
//          16-byte output rows out[i = 4 ig + q][c][o = 4 og .. +3] go to LDS
//          at [c][i][og] (one 16-byte slot each; the pitches of i and c are
//          padded as the planner finds free of bank conflicts for both phases);
//   write: the threads walk the slots in output order (o groups fastest,
//          then i or c, whichever is nearer the output's unit stride) and
//          store them: one store instruction covers a contiguous run of the
//          output as long as the dims allow.
// All LDS accesses are 16 bytes; no tables.
// one output row of a REG4 block (COPY or ADD; element stores when the
// output's rows are not vector-aligned)
template< typename T, int VB >
__device__ inline void reg4_store( PermArgs const & a, T * p, VecN< T, VB > w ) {
  if( a.vec_ok ) {
    if( a.add ) {
      VecN< T, VB > const l_old = *reinterpret_cast< VecN< T, VB > const * >( p );
#pragma unroll
      for( int l_r = 0; l_r < VB; l_r++ ) w.v[l_r] = Elem< T >::add( l_old.v[l_r], w.v[l_r] );
    }
    store_stream( reinterpret_cast< VecN< T, VB > * >( p ), w );
  }
  else {
#pragma unroll
    for( int l_r = 0; l_r < VB; l_r++ ) p[l_r] = a.add ? Elem< T >::add( p[l_r], w.v[l_r] ) : w.v[l_r];
  }
}

// Short unit-stride dims (REG4): VB x VB blocks (8 for bf16 when both dims
// allow it, else 4) transposed in registers, whole block rows
// exchanged through LDS.  i is the input's unit-stride dim, o the output's,
// c the dim walked next (the one that continues the input's run, or the
// output's); a workgroup takes all of i and o and c_chunk values of c.
//   read:  thread (ig, c, og) -- ig fastest -- loads the VB block rows
//          in[o = VB og + r][c][i = VB ig .. VB ig + VB - 1], r = 0..VB-1:
//          one load instruction of a wave covers one input row o over a
//          contiguous run of (c, i);
//   swap:  the block is transposed by renaming registers (for bf16 the
//          compiler packs the 16-bit halves with v_perm), and its VB output
//          rows out[i = VB ig + q][c][o = VB og .. +VB-1] go to LDS at
//          [c][i][og] (one slot each; the pitches of i and c are padded as the
//          planner finds free of bank conflicts for both phases);
//   write: the threads walk the slots in output order (o groups fastest,
//          then i or c, whichever is nearer the output's unit stride) and
//          store them: one store instruction covers a contiguous run of the
//          output as long as the dims allow.
// DIRECT: each thread stores its block rows itself, without the LDS exchange
// -- taken when the rows that one store instruction covers (o, continued by
// c) are whole 128-byte lines anyway.  No tables.
template< typename T, int VB, int CPT, int NT, bool DIRECT >
__global__ __launch_bounds__( NT )
void perm_reg4_kernel( PermArgs a ) {
  typedef VecN< T, VB > Row;
  extern __shared__ __attribute__( ( aligned( 16 ) ) ) char l_lds_raw[];
  Row * l_slots = reinterpret_cast< Row * >( l_lds_raw );
  int32_t const l_nig = int32_t( a.size_i / VB );
  int32_t const l_nog = int32_t( a.size_o / VB );
  int32_t const l_cw  = a.c_chunk / CPT;             // values of c per pass of the threads
  int32_t const l_ct  = a.c_chunk;                   // values of c per workgroup
  int32_t const l_pi  = a.slot_pi;                   // slots per i (nog + padding)
  int32_t const l_pc  = a.slot_pc;                   // slots per c (size_i * pi + padding)
  int32_t const l_used = l_nig * l_nog * l_cw;       // threads with a block

  uint32_t l_bid = blockIdx.x;
  int64_t const l_cbase = grid_digit( l_bid, a.c_nblk ) * l_ct;
  int64_t l_off_in  = 0;
  int64_t l_off_out = 0;
  for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
    int64_t const l_idx = grid_digit( l_bid, a.batch_size[l_d] );
    l_off_in  += l_idx * a.batch_s_in[l_d];
    l_off_out += l_idx * a.batch_s_out[l_d];
  }
  T const * l_in  = reinterpret_cast< T const * >( a.in ) + l_off_in;
  T       * l_out = reinterpret_cast< T * >( a.out ) + l_off_out;
  bool const l_active = int32_t( threadIdx.x ) < l_used;

  // read (all CPT passes' loads in flight together) + register transpose
  // + LDS (or, DIRECT, the stores)
  {
    int32_t l_x = threadIdx.x;
    int32_t const l_ig = l_x % l_nig;
    l_x /= l_nig;
    int32_t const l_cl = l_x % l_cw;
    int32_t const l_og = l_x / l_cw;
    T l_v[CPT][VB][VB];
    bool l_ok[CPT];
#pragma unroll
    for( int l_u = 0; l_u < CPT; l_u++ ) {
      int64_t const l_c = l_cbase + l_cl + l_u * l_cw;
      l_ok[l_u] = l_active && l_c < a.c_size;
      if( !l_ok[l_u] ) continue;
      T const * l_p = l_in + l_c * a.c_s_in + int64_t( VB * l_og ) * a.s_in_o + VB * l_ig;
      if( a.vec_ok ) {
#pragma unroll
        for( int l_r = 0; l_r < VB; l_r++ ) {
          Row const l_t = *reinterpret_cast< Row const * >( l_p + l_r * a.s_in_o );
#pragma unroll
          for( int l_q = 0; l_q < VB; l_q++ ) l_v[l_u][l_r][l_q] = l_t.v[l_q];
        }
      }
      else {
#pragma unroll
        for( int l_r = 0; l_r < VB; l_r++ )
#pragma unroll
          for( int l_q = 0; l_q < VB; l_q++ ) l_v[l_u][l_r][l_q] = l_p[l_r * a.s_in_o + l_q];
      }
    }
#pragma unroll
    for( int l_u = 0; l_u < CPT; l_u++ ) {
      if( !l_ok[l_u] ) continue;
#pragma unroll
      for( int l_q = 0; l_q < VB; l_q++ ) {
        Row l_w;
#pragma unroll
        for( int l_r = 0; l_r < VB; l_r++ ) l_w.v[l_r] = l_v[l_u][l_r][l_q];
        if constexpr( DIRECT ) {
          int64_t const l_c = l_cbase + l_cl + l_u * l_cw;
          reg4_store< T, VB >( a, l_out + l_c * a.c_s_out + int64_t( VB * l_ig + l_q ) * a.s_out_i + VB * l_og, l_w );
        }
        else {
          l_slots[( l_cl + l_u * l_cw ) * l_pc + ( VB * l_ig + l_q ) * l_pi + l_og] = l_w;
        }
      }
    }
  }
  if constexpr( DIRECT ) return;
  __syncthreads();
  // LDS -> output: the tile's slots in output order (o groups fastest, then
  // whichever of i and c has the smaller output stride), so that the 64
  // slots of one store instruction are as contiguous as the output allows
  {
    int32_t const l_si = int32_t( a.size_i );
    int32_t const l_nslots = l_si * l_ct * l_nog;
    bool const l_c_inner = a.c_s_out < a.s_out_i;
    for( int32_t l_s = threadIdx.x; l_s < l_nslots; l_s += NT ) {
      int32_t const l_og = l_s % l_nog;
      int32_t const l_s2 = l_s / l_nog;
      int32_t const l_cl = l_c_inner ? l_s2 % l_ct : l_s2 / l_si;
      int32_t const l_i  = l_c_inner ? l_s2 / l_ct : l_s2 % l_si;
      int64_t const l_c = l_cbase + l_cl;
      if( l_c >= a.c_size ) continue;
      reg4_store< T, VB >( a, l_out + l_c * a.c_s_out + int64_t( l_i ) * a.s_out_i + VB * l_og,
                           l_slots[l_cl * l_pc + l_i * l_pi + l_og] );
    }
  }
}

// Rows (ROWS): both tensors have the same unit-stride dim u, so the
// permutation moves whole rows of R = rows_g * VW elements.  x is the dim
// that continues the input's contiguous run (input stride R), y the one that
// continues the output's (output stride R).  A workgroup moves a tile of
// rows_ex x rows_ey rows: it reads the tile's ey input runs (ex rows each,
// contiguous), parks every chunk of VW elements in LDS at slot
// x * rows_pitch + y * g + c (the output's order) and writes the tile's ex
// output runs (ey rows each, contiguous).  Every index advances by adds (the
// step of the workgroup's threads is split into runs, rows and chunks once
// per tile); kPer chunks per thread are loaded before any is stored.
// raw bits of one chunk of B bytes (vector types stay in registers where
// arrays of the element structs were placed in scratch memory)
template< int B > struct RawChunk { typedef uint32_t type __attribute__( ( ext_vector_type( B / 4 ) ) ); };
template<> struct RawChunk< 4 > { typedef uint32_t type; };
template<> struct RawChunk< 2 > { typedef uint16_t type; };

template< typename T, int VW >
__global__ __launch_bounds__( kThreads )
void perm_rows_kernel( PermArgs a ) {
  typedef typename RawChunk< int( VW * sizeof( T ) ) >::type V;
  typedef VecN< T, VW > E;
  constexpr int kPer = 8;
  extern __shared__ __attribute__( ( aligned( 16 ) ) ) char l_lds_raw[];
  V * l_slots = reinterpret_cast< V * >( l_lds_raw );

  uint32_t l_bid = blockIdx.x;
  int64_t const l_bx = grid_digit( l_bid, a.rows_nbx );
  int64_t const l_by = grid_digit( l_bid, a.rows_nby );
  int64_t l_off_in = 0, l_off_out = 0;
  for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
    int64_t const l_idx = grid_digit( l_bid, a.batch_size[l_d] );
    l_off_in  += l_idx * a.batch_s_in[l_d];
    l_off_out += l_idx * a.batch_s_out[l_d];
  }
  int32_t const l_g  = a.rows_g;
  int64_t const l_x0 = int64_t( l_bx ) * a.rows_ex;
  int64_t const l_y0 = int64_t( l_by ) * a.rows_ey;
  int32_t const l_nx = int32_t( min( int64_t( a.rows_ex ), a.rows_nx - l_x0 ) );
  int32_t const l_ny = int32_t( min( int64_t( a.rows_ey ), a.rows_ny - l_y0 ) );
  int64_t const l_len = int64_t( l_g ) * VW;
  T const * l_in  = reinterpret_cast< T const * >( a.in ) + l_off_in + l_x0 * l_len + l_y0 * a.rows_s_in_y;
  T       * l_out = reinterpret_cast< T * >( a.out ) + l_off_out + l_y0 * l_len + l_x0 * a.rows_s_out_x;
  int32_t const l_pitch = a.rows_pitch;
  int32_t const l_tid   = threadIdx.x;

  // read: chunk j = (y, x, c), c fastest -- the tile's input runs in turn;
  // r = x * g + c is the chunk's place in its run
  int32_t const l_rrun = l_nx * l_g;
  int32_t const l_n    = l_ny * l_rrun;
  {
    // the step of kThreads chunks as (sy runs, sx rows, sc chunks)
    int32_t const l_sy = kThreads / l_rrun;
    int32_t const l_sx = ( kThreads - l_sy * l_rrun ) / l_g;
    int32_t const l_sc = kThreads - l_sy * l_rrun - l_sx * l_g;
    int32_t l_y = l_tid / l_rrun;
    int32_t l_x = ( l_tid - l_y * l_rrun ) / l_g;
    int32_t l_c = l_tid - l_y * l_rrun - l_x * l_g;
    for( int32_t l_j0 = 0; l_j0 < l_n; l_j0 += kPer * kThreads ) {
      V       l_v[kPer];
      int32_t l_s[kPer];
#pragma unroll
      for( int l_p = 0; l_p < kPer; l_p++ ) {
        l_s[l_p] = -1;
        if( l_j0 + l_p * kThreads + l_tid < l_n ) {
          l_v[l_p] = *reinterpret_cast< V const * >( l_in + int64_t( l_y ) * a.rows_s_in_y
                                                          + int64_t( l_x * l_g + l_c ) * VW );
          l_s[l_p] = l_x * l_pitch + l_y * l_g + l_c;
        }
        l_c += l_sc;
        l_x += l_sx;
        l_y += l_sy;
        if( l_c >= l_g )  { l_c -= l_g;  l_x++; }
        if( l_x >= l_nx ) { l_x -= l_nx; l_y++; }
      }
#pragma unroll
      for( int l_p = 0; l_p < kPer; l_p++ ) {
        if( l_s[l_p] >= 0 ) l_slots[l_s[l_p]] = l_v[l_p];
      }
    }
  }
  __syncthreads();
  // write: chunk j = (x, w), w = y * g + c fastest -- the tile's output runs
  // in turn
  int32_t const l_wrun = l_ny * l_g;
  {
    int32_t const l_sx = kThreads / l_wrun;
    int32_t const l_sw = kThreads - l_sx * l_wrun;
    int32_t l_x = l_tid / l_wrun;
    int32_t l_w = l_tid - l_x * l_wrun;
    for( int32_t l_j0 = 0; l_j0 < l_n; l_j0 += kPer * kThreads ) {
      V       l_v[kPer];
      int64_t l_o[kPer];
#pragma unroll
      for( int l_p = 0; l_p < kPer; l_p++ ) {
        l_o[l_p] = -1;
        if( l_j0 + l_p * kThreads + l_tid < l_n ) {
          l_v[l_p] = l_slots[l_x * l_pitch + l_w];
          l_o[l_p] = int64_t( l_x ) * a.rows_s_out_x + int64_t( l_w ) * VW;
        }
        l_w += l_sw;
        l_x += l_sx;
        if( l_w >= l_wrun ) { l_w -= l_wrun; l_x++; }
      }
#pragma unroll
      for( int l_p = 0; l_p < kPer; l_p++ ) {
        if( l_o[l_p] < 0 ) continue;
        V * l_ptr = reinterpret_cast< V * >( l_out + l_o[l_p] );
        if( a.add ) {
          E const l_old = __builtin_bit_cast( E, *l_ptr );
          E       l_sum = __builtin_bit_cast( E, l_v[l_p] );
#pragma unroll
          for( int l_e = 0; l_e < VW; l_e++ ) l_sum.v[l_e] = Elem< T >::add( l_old.v[l_e], l_sum.v[l_e] );
          *l_ptr = __builtin_bit_cast( V, l_sum );
        }
        else {
          __builtin_nontemporal_store( l_v[l_p], l_ptr );
        }
      }
    }
  }
}

// One thread per VW consecutive output elements of the innermost dim.
// Dims are (outer -> inner) in a.batch_*; for VW > 1 the innermost dim has
// unit stride in both tensors and a size divisible by VW (VW elements are one
// 16-byte vector for bf16 and fp32, 32 bytes for fp64).  I is the type of
// the element index the coordinates are decoded from: uint32_t when the
// element count fits it (32-bit division), else uint64_t.
template< typename T, int VW, bool FILL, typename I >
__global__ __launch_bounds__( kThreads )
void perm_gather_kernel( PermArgs a ) {
  typedef VecN< T, VW > V;
  int64_t const l_num_items = a.num_elements / VW;
  for( int64_t l_item = int64_t( blockIdx.x ) * kThreads + threadIdx.x;
       l_item < l_num_items;
       l_item += int64_t( gridDim.x ) * kThreads ) {
    I l_rem = I( l_item * VW );
    int64_t l_off_in  = 0;
    int64_t l_off_out = 0;
    for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
      I const l_sz  = I( a.batch_size[l_d] );
      I const l_q   = l_rem / l_sz;
      int64_t const l_idx = int64_t( l_rem - l_q * l_sz );
      l_rem = l_q;
      l_off_in  += l_idx * a.batch_s_in[l_d];
      l_off_out += l_idx * a.batch_s_out[l_d];
    }
    T * l_out = reinterpret_cast< T * >( a.out ) + l_off_out;
    if( FILL ) {
      V l_z;
#pragma unroll
      for( int l_e = 0; l_e < VW; l_e++ ) l_z.v[l_e] = T( 0 );
      *reinterpret_cast< V * >( l_out ) = l_z;
      continue;
    }
    T const * l_in = reinterpret_cast< T const * >( a.in ) + l_off_in;
    V l_v = *reinterpret_cast< V const * >( l_in );
    if( a.add ) {
      V const l_old = *reinterpret_cast< V const * >( l_out );
#pragma unroll
      for( int l_e = 0; l_e < VW; l_e++ ) l_v.v[l_e] = Elem< T >::add( l_old.v[l_e], l_v.v[l_e] );
    }
    *reinterpret_cast< V * >( l_out ) = l_v;
  }
}

// REG4 launch: every (block side, passes, threads, direct) variant from one table
template< typename T, int VB >
int launch_reg4( PermutePlan const & p, PermArgs const & a, int64_t blocks, hipStream_t stream ) {
  std::size_t const l_lds = std::size_t( a.c_chunk ) * a.slot_pc * VB * sizeof( T );
  dim3 const l_grid( (uint32_t) blocks );
  auto launch = [&]( auto i_kernel, int i_threads, bool i_direct ) {
    hipLaunchKernelGGL( i_kernel, l_grid, dim3( i_threads ), i_direct ? 0 : l_lds, stream, a );
    return int( ETIR_SUCCESS );
  };
  bool const l_d = p.reg4_direct;
  if( p.reg4_cpt == 4 )                        return launch( perm_reg4_kernel< T, VB, 4, kThreads, false >, kThreads, false );
  if( p.reg4_cpt == 2 )                        return launch( perm_reg4_kernel< T, VB, 2, kThreads, false >, kThreads, false );
  if( p.reg4_threads == 64 && l_d )            return launch( perm_reg4_kernel< T, VB, 1, 64, true >, 64, true );
  if( p.reg4_threads == 64 )                   return launch( perm_reg4_kernel< T, VB, 1, 64, false >, 64, false );
  if( p.reg4_threads == 128 && l_d )           return launch( perm_reg4_kernel< T, VB, 1, 128, true >, 128, true );
  if( p.reg4_threads == 128 )                  return launch( perm_reg4_kernel< T, VB, 1, 128, false >, 128, false );
  if( p.reg4_threads == kThreads && l_d )      return launch( perm_reg4_kernel< T, VB, 1, kThreads, true >, kThreads, true );
  if( p.reg4_threads == kThreads )             return launch( perm_reg4_kernel< T, VB, 1, kThreads, false >, kThreads, false );
  if( p.reg4_threads == 512 && l_d )           return launch( perm_reg4_kernel< T, VB, 1, 512, true >, 512, true );
  if( p.reg4_threads == 512 )                  return launch( perm_reg4_kernel< T, VB, 1, 512, false >, 512, false );
  return fail( ETIR_UNDEFINED_ERROR, "permute: no REG4 kernel for this workgroup size" );
}

template< typename X > struct IdxTag { typedef X type; };

template< typename T >
int launch_typed( PermutePlan const & p,
                  PermArgs          & a,
                  hipStream_t         stream ) {
  if( p.mode == PermMode::TILED ) {
    int64_t l_blocks = a.num_batch_total;
    for( int l_k = 0; l_k < a.tile_nd; l_k++ ) l_blocks *= a.tile_nblk[l_k];
    if( l_blocks > 0x7fffffffLL ) {
      return fail( ETIR_UNDEFINED_ERROR, "permute: grid too large" );
    }
    std::size_t const l_lds = std::size_t( a.tile_n + ( a.tile_n >> 6 ) * a.tile_pad ) * sizeof( T );
    if( p.tile_vw == 4 ) {
      hipLaunchKernelGGL( ( perm_tiled_kernel< T, 4 > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), l_lds, stream, a );
    }
    else {
      hipLaunchKernelGGL( ( perm_tiled_kernel< T, 1 > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), l_lds, stream, a );
    }
  }
  else if( p.mode == PermMode::REG4 ) {
    a.c_nblk = ( a.c_size + a.c_chunk - 1 ) / a.c_chunk;
    int64_t const l_blocks = a.c_nblk * a.num_batch_total;
    if( l_blocks > 0x7fffffffLL ) {
      return fail( ETIR_UNDEFINED_ERROR, "permute: grid too large" );
    }
    // the launch's own errors (no kernel for the workgroup size) return at
    // once; launch failures fall through to the shared check below
    int l_rc = ETIR_SUCCESS;
    if constexpr( sizeof( T ) == 2 ) {
      if( p.reg4_vb == 8 ) l_rc = launch_reg4< T, 8 >( p, a, l_blocks, stream );
      else                 l_rc = launch_reg4< T, 4 >( p, a, l_blocks, stream );
    }
    else {
      l_rc = launch_reg4< T, 4 >( p, a, l_blocks, stream );
    }
    if( l_rc != ETIR_SUCCESS ) return l_rc;
  }
  else if( p.mode == PermMode::ROWS ) {
    int64_t const l_blocks = a.rows_nbx * a.rows_nby * a.num_batch_total;
    if( l_blocks > 0x7fffffffLL ) {
      return fail( ETIR_UNDEFINED_ERROR, "permute: grid too large" );
    }
    std::size_t const l_lds = std::size_t( a.rows_ex ) * a.rows_pitch * p.rows_vw * sizeof( T );
    auto launch = [&]( auto i_vw ) {
      constexpr int l_vw = decltype( i_vw )::value;
      hipLaunchKernelGGL( ( perm_rows_kernel< T, l_vw > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), l_lds, stream, a );
    };
    int64_t const l_cb = p.rows_vw * int64_t( sizeof( T ) );
    if constexpr( sizeof( T ) <= 8 ) {
      if( l_cb == 16 ) launch( std::integral_constant< int, int( 16 / sizeof( T ) ) >() );
    }
    if constexpr( sizeof( T ) <= 4 ) {
      if( l_cb == 8 ) launch( std::integral_constant< int, int( 8 / sizeof( T ) ) >() );
    }
    if constexpr( sizeof( T ) == 2 ) {
      if( l_cb == 4 ) launch( std::integral_constant< int, 2 >() );
    }
    if( p.rows_vw == 1 ) launch( std::integral_constant< int, 1 >() );
  }
  else if( p.mode == PermMode::TRANSPOSE ) {
    int64_t l_blocks = a.tiles_i * a.tiles_o * a.num_batch_total;
    if( l_blocks > 0x7fffffffLL ) {
      return fail( ETIR_UNDEFINED_ERROR, "permute: grid too large" );
    }
    dim3 const l_g( (uint32_t) l_blocks );
    if( p.tr_shape == 3 || p.tr_shape == 4 ) {
      if constexpr( sizeof( T ) == 2 ) {
        auto go = [&]( auto to_c, auto vec_c ) {
          if( a.o1_size > 0 ) {
            hipLaunchKernelGGL( ( perm_transpose16_kernel< T, 128, decltype( to_c )::value, decltype( vec_c )::value,
                                                           true > ), l_g, dim3( kThreads ), 0, stream, a );
          }
          else {
            hipLaunchKernelGGL( ( perm_transpose16_kernel< T, 128, decltype( to_c )::value, decltype( vec_c )::value,
                                                           false > ), l_g, dim3( kThreads ), 0, stream, a );
          }
        };
        std::integral_constant< int, 64 > const l_to64{};
        std::integral_constant< int, 32 > const l_to32{};
        if( p.tr_shape == 3 ) {
          if( a.vec_ok ) go( l_to64, std::true_type() );
          else           go( l_to64, std::false_type() );
        }
        else {
          if( a.vec_ok ) go( l_to32, std::true_type() );
          else           go( l_to32, std::false_type() );
        }
      }
      else {
        return fail( ETIR_UNDEFINED_ERROR, "permute: 16-byte transpose tile for a non-2-byte type" );
      }
    }
    else if( p.tr_shape == 1 ) hipLaunchKernelGGL( ( perm_transpose_kernel< T, 128, 32 > ), l_g, dim3( kThreads ), 0, stream, a );
    else if( p.tr_shape == 2 ) hipLaunchKernelGGL( ( perm_transpose_kernel< T, 32, 128 > ), l_g, dim3( kThreads ), 0, stream, a );
    else                       hipLaunchKernelGGL( ( perm_transpose_kernel< T, 64, 64 > ), l_g, dim3( kThreads ), 0, stream, a );
  }
  else {
    // bf16 moves 8 elements (16 bytes) per vector where the planner allows it
    int const l_vw = !a.vec_ok ? 1 : ( a.vec_wide && sizeof( T ) == 2 ? 8 : 4 );
    int64_t l_items = a.num_elements / l_vw;
    int64_t l_blocks = ( l_items + kThreads - 1 ) / kThreads;
    l_blocks = std::min< int64_t >( l_blocks, 65536 );
    if( l_blocks < 1 ) l_blocks = 1;
    dim3 const l_g( (uint32_t) l_blocks );
    auto launch = [&]( auto i_fill, auto i_idx ) {
      constexpr bool l_fill = decltype( i_fill )::value;
      typedef typename decltype( i_idx )::type I;
      if( l_vw == 8 )      hipLaunchKernelGGL( ( perm_gather_kernel< T, 8, l_fill, I > ), l_g, dim3( kThreads ), 0, stream, a );
      else if( l_vw == 4 ) hipLaunchKernelGGL( ( perm_gather_kernel< T, 4, l_fill, I > ), l_g, dim3( kThreads ), 0, stream, a );
      else                 hipLaunchKernelGGL( ( perm_gather_kernel< T, 1, l_fill, I > ), l_g, dim3( kThreads ), 0, stream, a );
    };
    bool const l_small = a.num_elements <= int64_t( UINT32_MAX );
    if( p.mode == PermMode::FILL ) {
      if( l_small ) launch( std::true_type(), IdxTag< uint32_t >() );
      else          launch( std::true_type(), IdxTag< uint64_t >() );
    }
    else {
      if( l_small ) launch( std::false_type(), IdxTag< uint32_t >() );
      else          launch( std::false_type(), IdxTag< uint64_t >() );
    }
  }
  hipError_t l_err = hipGetLastError();
  if( l_err != hipSuccess ) {
    return fail( ETIR_UNDEFINED_ERROR, std::string( "permute launch failed: " ) + hipGetErrorString( l_err ) );
  }
  return ETIR_SUCCESS;
}

// ROWS configuration for a permutation whose tensors share their
// unit-stride dim dim_u (plan.size/s_in/s_out set); false when the rows are
// long (the vector copy moves them as well), or no dim continues the input's
// or the output's run past the rows.
bool plan_rows( PermutePlan & plan, int dim_u ) {
  if( char const * l_env = std::getenv( "ETIR_PERM_ROWS" ) ) {
    if( std::atoi( l_env ) == 0 ) return false;
  }
  // rows from 256 bytes on (bf16: 128) move as fast with the vector copy
  // (fp32 abcd->cabd 16,32,256,64: 68.5 % copy against 64.2 % ROWS; bf16
  // 16,32,256,64: 65 % against 52-56 %)
  int64_t l_max_bytes = plan.elem_bytes == 2 ? 128 : 256;
  if( char const * l_env = std::getenv( "ETIR_PERM_ROWS_MAX_BYTES" ) ) l_max_bytes = std::atoll( l_env );
  int const     l_n    = plan.num_dims;
  int64_t const l_esz  = plan.elem_bytes;
  int64_t const l_len  = plan.size[dim_u];
  int64_t const l_rowb = l_len * l_esz;
  if( l_rowb < 16 || l_rowb >= l_max_bytes ) return false;
  int l_x = -1, l_y = -1;
  for( int l_d = 0; l_d < l_n; l_d++ ) {
    if( l_d == dim_u ) continue;
    if( plan.s_in[l_d]  == l_len && l_x < 0 ) l_x = l_d;
    if( plan.s_out[l_d] == l_len && l_y < 0 ) l_y = l_d;
  }
  if( l_x < 0 || l_y < 0 || l_x == l_y ) return false;
  // chunk: the widest of 16, 8, 4 bytes that divides the row and every stride
  auto fits = [&]( int64_t vw ) {
    if( l_len % vw != 0 ) return false;
    for( int l_d = 0; l_d < l_n; l_d++ ) {
      if( l_d != dim_u && ( plan.s_in[l_d] % vw != 0 || plan.s_out[l_d] % vw != 0 ) ) return false;
    }
    return true;
  };
  int64_t l_vw = 16 / l_esz;
  while( l_vw > 1 && !( l_vw * l_esz >= 4 && fits( l_vw ) ) ) l_vw /= 2;
  if( !fits( l_vw ) ) l_vw = 1;
  int64_t const l_g  = l_len / l_vw;
  int64_t const l_cb = l_vw * l_esz;
  int64_t const l_nx = plan.size[l_x], l_ny = plan.size[l_y];
  // tile extents: at most 18 KB of rows and 1536 chunks (fp32 cabd-like
  // shapes: 12-18 KB tiles 74-81 % of HBM peak, 24-32 KB 64-74 %, 6 KB
  // 50-55 %; bf16 with 8-byte chunks: 1152-1536 chunks 70 %, 2304 chunks
  // 58-61 %), runs of at least 256 bytes (or the whole dim), the fewest
  // passes of the threads over all tiles, with two passes' worth added per
  // tile for its index decode and barrier and half as much again per side
  // whose runs are not whole 128-byte lines (bf16 abc->bac 2048,1024,12:
  // 32 x 16 rows, runs of 768 and 384 bytes, 70 %; 22 x 23 rows, 528 and 552
  // bytes, 59 %)
  int64_t l_ex = 0, l_ey = 0;
  {
    int64_t l_best = -1;
    int64_t const l_rx = std::min< int64_t >( 256, l_nx * l_rowb ), l_ry = std::min< int64_t >( 256, l_ny * l_rowb );
    for( int64_t l_tx = 1; l_tx <= std::min< int64_t >( l_nx, 256 ); l_tx++ ) {
      if( l_tx * l_rowb < l_rx ) continue;
      for( int64_t l_ty = 1; l_ty <= std::min< int64_t >( l_ny, 256 ); l_ty++ ) {
        if( l_tx * l_ty * l_rowb > 18432 || l_tx * l_ty * l_g > 1536 ) break;
        if( l_ty * l_rowb < l_ry ) continue;
        int64_t const l_tiles = ( ( l_nx + l_tx - 1 ) / l_tx ) * ( ( l_ny + l_ty - 1 ) / l_ty );
        int64_t l_cost = l_tiles * ( ( l_tx * l_ty * l_g + kThreads - 1 ) / kThreads + 2 ) * 4;
        if( l_tx < l_nx && ( l_tx * l_rowb ) % 128 != 0 ) l_cost += l_cost / 2;
        if( l_ty < l_ny && ( l_ty * l_rowb ) % 128 != 0 ) l_cost += l_cost / 2;
        if( l_best < 0 || l_cost < l_best || ( l_cost == l_best && l_tx * l_ty > l_ex * l_ey ) ) {
          l_best = l_cost;
          l_ex = l_tx;
          l_ey = l_ty;
        }
      }
    }
  }
  if( l_ex == 0 ) return false;
  // LDS pitch: simulate both phases' accesses of a full tile (128 bytes of
  // lanes per LDS cycle, 64 four-byte banks) and take the padding with the
  // fewest conflicts
  {
    int64_t const l_lanes  = std::max< int64_t >( 1, 128 / l_cb );
    int64_t const l_words  = std::max< int64_t >( 1, l_cb / 4 );
    int64_t const l_groups = 64 / l_words;
    int64_t const l_n_ch   = l_ex * l_ey * l_g;
    int64_t l_best = -1;
    for( int64_t l_pad = 0; l_pad < 16; l_pad++ ) {
      int64_t const l_pitch = l_ey * l_g + l_pad;
      if( l_pad > 0 && l_ex * l_pitch * l_cb > 40960 ) break;
      int64_t l_cost = 0;
      for( int l_phase = 0; l_phase < 2; l_phase++ ) {
        for( int64_t l_j0 = 0; l_j0 < l_n_ch; l_j0 += l_lanes ) {
          int l_cnt[64] = { 0 };
          int l_mx = 0;
          for( int64_t l_j = l_j0; l_j < std::min( l_n_ch, l_j0 + l_lanes ); l_j++ ) {
            int64_t l_slot;
            if( l_phase == 0 ) {
              int64_t const l_yy = l_j / ( l_ex * l_g ), l_r = l_j % ( l_ex * l_g );
              l_slot = ( l_r / l_g ) * l_pitch + l_yy * l_g + l_r % l_g;
            }
            else {
              l_slot = ( l_j / ( l_ey * l_g ) ) * l_pitch + l_j % ( l_ey * l_g );
            }
            int64_t const l_bank = ( l_cb >= 4 ? l_slot : l_slot * l_cb / 4 ) % l_groups;
            l_mx = std::max( l_mx, ++l_cnt[l_bank] );
          }
          l_cost += l_mx;
        }
      }
      if( l_best < 0 || l_cost < l_best ) {
        l_best = l_cost;
        plan.args.rows_pitch = int32_t( l_pitch );
      }
    }
  }
  PermArgs & a = plan.args;
  plan.mode     = PermMode::ROWS;
  plan.rows_vw  = int32_t( l_vw );
  plan.rows_len = l_len;
  a.rows_g       = int32_t( l_g );
  a.rows_ex      = int32_t( l_ex );
  a.rows_ey      = int32_t( l_ey );
  a.rows_nx      = l_nx;
  a.rows_ny      = l_ny;
  a.rows_nbx     = ( l_nx + l_ex - 1 ) / l_ex;
  a.rows_nby     = ( l_ny + l_ey - 1 ) / l_ey;
  a.rows_s_in_y  = plan.s_in[l_y];
  a.rows_s_out_x = plan.s_out[l_x];
  a.num_batch = 0;
  a.num_batch_total = 1;
  for( int l_d = 0; l_d < l_n; l_d++ ) {
    if( l_d == dim_u || l_d == l_x || l_d == l_y ) continue;
    a.batch_size[a.num_batch]  = plan.size[l_d];
    a.batch_s_in[a.num_batch]  = plan.s_in[l_d];
    a.batch_s_out[a.num_batch] = plan.s_out[l_d];
    a.num_batch_total *= plan.size[l_d];
    a.num_batch++;
  }
  a.vec_ok = l_vw > 1 ? 1 : 0;
  return true;
}

// TILED configuration of a fused permutation (plan.size/s_in/s_out set, dim_i /
// dim_o the unit-stride dims of input and output); false if the shape does
// not fit it (then the other modes apply).
bool plan_tiled( PermutePlan & plan, int dim_i, int dim_o ) {
  int const l_n = plan.num_dims;
  int64_t const l_esz = plan.elem_bytes;
  // innermost contiguous run of one tensor, grown from its unit-stride dim
  auto run = [&]( int unit, int64_t const * st ) {
    std::vector< int > l_r{ unit };
    int64_t l_prod = plan.size[unit];
    while( l_prod < kTile && l_r.size() < 2 ) {
      int l_next = -1;
      for( int l_d = 0; l_d < l_n; l_d++ ) {
        if( std::find( l_r.begin(), l_r.end(), l_d ) == l_r.end() && st[l_d] == l_prod ) {
          l_next = l_d;
          break;
        }
      }
      if( l_next < 0 ) break;
      l_r.push_back( l_next );
      l_prod *= plan.size[l_next];
    }
    return l_r;
  };
  std::vector< int > const l_ri = run( dim_i, plan.s_in );
  std::vector< int > const l_ro = run( dim_o, plan.s_out );
  // extent a dim needs in a run: whole for an inner dim, enough for 64
  // elements for the run's outermost dim
  auto need = [&]( std::vector< int > const & r, int d ) -> int64_t {
    int64_t l_p = 1;
    for( std::size_t l_k = 0; l_k < r.size(); l_k++ ) {
      if( r[l_k] == d ) {
        return ( l_k + 1 == r.size() ) ? std::min< int64_t >( plan.size[d], ( kTile + l_p - 1 ) / l_p )
                                       : plan.size[d];
      }
      l_p *= plan.size[r[l_k]];
    }
    return 0;
  };
  std::vector< int > l_td;
  for( int l_d : l_ri ) l_td.push_back( l_d );
  for( int l_d : l_ro ) if( std::find( l_td.begin(), l_td.end(), l_d ) == l_td.end() ) l_td.push_back( l_d );
  int const l_nt = (int) l_td.size();
  // one tile dim (a shared unit-stride dim that no run extends): the
  // vectorised copy moves the same runs without the tables
  if( l_nt < 2 || l_nt > kPermTileDims ) return false;
  std::vector< int64_t > l_e( l_nt );
  for( int l_k = 0; l_k < l_nt; l_k++ ) {
    l_e[l_k] = std::max( need( l_ri, l_td[l_k] ), need( l_ro, l_td[l_k] ) );
    if( l_e[l_k] > 255 ) return false;
  }
  auto tile_n = [&]() {
    int64_t l_t = 1;
    for( int64_t l_x : l_e ) l_t *= l_x;
    return l_t;
  };
  // tiles of kPermTileMax elements where the dims allow (grow the outermost
  // run dims): small tiles leave each workgroup too little work
  // first the run needs alone may exceed the limit: halve the largest extent,
  // the unit-stride dims' last (their multiples of 4 keep 16-byte accesses)
  int const l_ui = (int) ( std::find( l_td.begin(), l_td.end(), dim_i ) - l_td.begin() );
  int const l_uo = (int) ( std::find( l_td.begin(), l_td.end(), dim_o ) - l_td.begin() );
  while( tile_n() > kPermTileMax ) {
    int l_big = -1;
    for( int l_k = 0; l_k < l_nt; l_k++ ) {
      if( l_k == l_ui || l_k == l_uo || l_e[l_k] <= 1 ) continue;
      if( l_big < 0 || l_e[l_k] > l_e[l_big] ) l_big = l_k;
    }
    if( l_big < 0 ) l_big = ( l_e[l_ui] >= l_e[l_uo] ) ? l_ui : l_uo;
    if( l_e[l_big] <= 1 ) return false;
    l_e[l_big] = ( l_e[l_big] + 1 ) / 2;
  }
  // then grow the outermost run dims while the tile stays within the limit
  bool l_grew = true;
  while( l_grew ) {
    l_grew = false;
    for( int l_k = l_nt - 1; l_k >= 0; l_k-- ) {
      int64_t const l_cap = std::min< int64_t >( plan.size[l_td[l_k]], 128 );
      int64_t const l_new = std::min( l_cap, 2 * l_e[l_k] );
      if( l_new > l_e[l_k] && tile_n() / l_e[l_k] * l_new <= kPermTileMax ) {
        l_e[l_k] = l_new;
        l_grew = true;
      }
    }
  }
  int64_t const l_tn = tile_n();

  // element orders: input order (tile dims by ascending input stride) and
  // output order (by ascending output stride), first dim fastest
  std::vector< int > l_oin( l_nt ), l_oout( l_nt );
  for( int l_k = 0; l_k < l_nt; l_k++ ) l_oin[l_k] = l_oout[l_k] = l_k;
  std::stable_sort( l_oin.begin(), l_oin.end(),
                    [&]( int x, int y ) { return plan.s_in[l_td[x]] < plan.s_in[l_td[y]]; } );
  std::stable_sort( l_oout.begin(), l_oout.end(),
                    [&]( int x, int y ) { return plan.s_out[l_td[x]] < plan.s_out[l_td[y]]; } );
  auto coords_of = [&]( int64_t lin, std::vector< int > const & order, int64_t * c ) {
    for( int l_k : order ) {
      c[l_k] = lin % l_e[l_k];
      lin /= l_e[l_k];
    }
  };
  auto t_of = [&]( int64_t const * c ) {   // input-order index of coordinates
    int64_t l_t = 0;
    for( int l_j = l_nt - 1; l_j >= 0; l_j-- ) l_t = l_t * l_e[l_oin[l_j]] + c[l_oin[l_j]];
    return l_t;
  };

  // LDS padding after every 64 elements: the one with the fewest bank
  // conflicts of the output-order reads (64 lanes per wave, 4-byte banks)
  std::vector< int64_t > l_tw( (std::size_t) l_tn );
  {
    int64_t l_c[kPermTileDims];
    for( int64_t l_u = 0; l_u < l_tn; l_u++ ) {
      coords_of( l_u, l_oout, l_c );
      l_tw[l_u] = t_of( l_c );
    }
  }
  int l_pad = 0;
  int64_t l_best = -1;
  for( int l_cand : { 0, 1, 2, 3, 4, 5, 7, 8, 9, 16, 17, 33 } ) {
    if( ( l_tn + ( l_tn >> 6 ) * l_cand ) * l_esz > 48 * 1024 ) break;
    int64_t l_cost = 0;
    for( int64_t l_w = 0; l_w < l_tn; l_w += 64 ) {
      std::vector< std::vector< int64_t > > l_words( 64 );
      for( int64_t l_u = l_w; l_u < std::min< int64_t >( l_w + 64, l_tn ); l_u++ ) {
        int64_t const l_t = l_tw[l_u];
        int64_t const l_word = ( ( l_t + ( l_t >> 6 ) * l_cand ) * l_esz ) / 4;
        std::vector< int64_t > & l_b = l_words[l_word % 64];
        if( std::find( l_b.begin(), l_b.end(), l_word ) == l_b.end() ) l_b.push_back( l_word );
      }
      std::size_t l_max = 1;
      for( auto const & l_b : l_words ) l_max = std::max( l_max, l_b.size() );
      l_cost += (int64_t) l_max;
    }
    if( l_best < 0 || l_cost < l_best ) {
      l_best = l_cost;
      l_pad = l_cand;
    }
  }

  // entries of 4 elements when the innermost run dims of both tensors (the
  // first dims of both orders) hold whole groups of 4, else of 1
  int const l_ki = (int) ( std::find( l_td.begin(), l_td.end(), dim_i ) - l_td.begin() );
  int const l_ko = (int) ( std::find( l_td.begin(), l_td.end(), dim_o ) - l_td.begin() );
  int const l_vw = (    l_e[l_ki] % 4 == 0 && plan.size[dim_i] % 4 == 0
                     && l_e[l_ko] % 4 == 0 && plan.size[dim_o] % 4 == 0 ) ? 4 : 1;
  int64_t const l_nv = l_tn / l_vw;
  // input-order step between neighbours along the output's unit-stride dim
  int64_t l_tstep = 1;
  for( int l_k : l_oin ) {
    if( l_k == l_ko ) break;
    l_tstep *= l_e[l_k];
  }

  // tables: write entries {output offset, first input-order index} (int2),
  // read offsets, and the packed coordinates of both (edge tiles only)
  std::vector< int32_t > l_w( 2 * l_nv ), l_r( l_nv ), l_rc( l_nv ), l_wc( l_nv );
  int64_t l_c[kPermTileDims];
  auto offset_pack = [&]( int64_t const * st, int64_t & off, uint32_t & pack ) {
    off = 0;
    pack = 0;
    for( int l_k = 0; l_k < l_nt; l_k++ ) {
      off += l_c[l_k] * st[l_td[l_k]];
      pack |= uint32_t( l_c[l_k] ) << ( 8 * l_k );
    }
  };
  for( int64_t l_j = 0; l_j < l_nv; l_j++ ) {
    coords_of( l_vw * l_j, l_oin, l_c );
    int64_t l_off;
    uint32_t l_pack;
    offset_pack( plan.s_in, l_off, l_pack );
    if( l_off > std::numeric_limits< int32_t >::max() ) return false;
    l_r[l_j]  = (int32_t) l_off;
    l_rc[l_j] = (int32_t) l_pack;
  }
  for( int64_t l_j = 0; l_j < l_nv; l_j++ ) {
    coords_of( l_vw * l_j, l_oout, l_c );
    int64_t l_off;
    uint32_t l_pack;
    offset_pack( plan.s_out, l_off, l_pack );
    if( l_off > std::numeric_limits< int32_t >::max() ) return false;
    l_w[2 * l_j]     = (int32_t) l_off;
    l_w[2 * l_j + 1] = (int32_t) l_tw[l_vw * l_j];
    l_wc[l_j]        = (int32_t) l_pack;
  }
  // one blob: write entries first (8-byte aligned), then the int32 arrays
  std::vector< int32_t > l_blob;
  l_blob.reserve( 5 * l_nv );
  for( auto const * l_v : { &l_w, &l_r, &l_rc, &l_wc } ) l_blob.insert( l_blob.end(), l_v->begin(), l_v->end() );
  std::size_t const l_bytes = l_blob.size() * sizeof( int32_t );
  void * l_dev = nullptr;
  if( hipMalloc( &l_dev, l_bytes ) != hipSuccess ) {
    (void) hipGetLastError();
    return false;
  }
  if( hipMemcpy( l_dev, l_blob.data(), l_bytes, hipMemcpyHostToDevice ) != hipSuccess ) {
    (void) hipGetLastError();
    (void) hipFree( l_dev );
    return false;
  }

  plan.mode = PermMode::TILED;
  plan.d_tables = l_dev;
  plan.tile_vw = l_vw;
  PermArgs & a = plan.args;
  a.tile_nd = l_nt;
  a.tile_n = (int32_t) l_tn;
  a.tile_pad = l_pad;
  a.tile_t_step = (int32_t) l_tstep;
  for( int l_k = 0; l_k < l_nt; l_k++ ) {
    int const l_d = l_td[l_k];
    a.tile_size[l_k]  = plan.size[l_d];
    a.tile_ext[l_k]   = l_e[l_k];
    a.tile_s_in[l_k]  = plan.s_in[l_d];
    a.tile_s_out[l_k] = plan.s_out[l_d];
    a.tile_nblk[l_k]  = ( plan.size[l_d] + l_e[l_k] - 1 ) / l_e[l_k];
  }
  int32_t const * l_tabs = static_cast< int32_t const * >( l_dev );
  a.tab_w  = l_tabs;
  a.tab_r  = l_tabs + 2 * l_nv;
  a.tab_rc = l_tabs + 3 * l_nv;
  a.tab_wc = l_tabs + 4 * l_nv;
  a.num_batch = 0;
  a.num_batch_total = 1;
  for( int l_d = 0; l_d < l_n; l_d++ ) {
    if( std::find( l_td.begin(), l_td.end(), l_d ) != l_td.end() ) continue;
    a.batch_size[a.num_batch]  = plan.size[l_d];
    a.batch_s_in[a.num_batch]  = plan.s_in[l_d];
    a.batch_s_out[a.num_batch] = plan.s_out[l_d];
    a.num_batch_total *= plan.size[l_d];
    a.num_batch++;
  }
  // 16-byte accesses: entries of 4 and every other stride a multiple of 4
  // (the pointers' alignment is checked at launch)
  a.vec_ok = ( l_vw == 4 ) ? 1 : 0;
  for( int l_d = 0; l_d < l_n && a.vec_ok; l_d++ ) {
    if( l_d != dim_i && plan.s_in[l_d] % 4 != 0 ) a.vec_ok = 0;
    if( l_d != dim_o && plan.s_out[l_d] % 4 != 0 ) a.vec_ok = 0;
  }
  return true;
}

}  // namespace

void release_permute( PermutePlan & plan ) {
  if( plan.d_tables != nullptr ) {
    (void) hipFree( plan.d_tables );
    plan.d_tables = nullptr;
  }
}

int plan_permute( int64_t         num_dims,
                  int64_t const * sizes,
                  int64_t const * strides_in,
                  int64_t const * strides_out,
                  int32_t         dtype,
                  int32_t         ktype,
                  PermutePlan   & plan ) {
  plan = PermutePlan();
  if( dtype != ETIR_FP32 && dtype != ETIR_FP64 && dtype != ETIR_BF16 ) {
    return fail( ETIR_INVALID_DTYPE, "permute: unsupported dtype" );
  }
  if( ktype != ETIR_KTYPE_COPY && ktype != ETIR_KTYPE_ZERO && ktype != ETIR_KTYPE_ADD ) {
    return fail( ETIR_INVALID_KTYPE, "permute: ktype must be COPY, ZERO or ADD" );
  }
  if( num_dims < 0 || ( num_dims > 0 && ( sizes == nullptr || strides_out == nullptr ) ) ) {
    return fail( ETIR_COMPILATION_FAILED, "permute: invalid dimension arrays" );
  }
  if( ktype != ETIR_KTYPE_ZERO && num_dims > 0 && strides_in == nullptr ) {
    return fail( ETIR_COMPILATION_FAILED, "permute: input strides missing" );
  }
  plan.dtype = dtype;
  plan.ktype = ktype;
  plan.elem_bytes = dtype_bytes( dtype );

  // collect non-trivial dims
  struct D { int64_t size, si, so; };
  std::vector< D > l_dims;
  int64_t l_num = 1;
  for( int64_t l_di = 0; l_di < num_dims; l_di++ ) {
    if( sizes[l_di] < 0 ) {
      return fail( ETIR_COMPILATION_FAILED, "permute: negative size" );
    }
    l_num *= sizes[l_di];
    if( sizes[l_di] == 1 ) continue;
    int64_t l_si = ( ktype == ETIR_KTYPE_ZERO ) ? 0 : strides_in[l_di];
    l_dims.push_back( { sizes[l_di], l_si, strides_out[l_di] } );
  }
  plan.num_elements = l_num;

  // order by output stride (outer -> inner), keep the given order on ties
  std::stable_sort( l_dims.begin(), l_dims.end(),
                    []( D const & x, D const & y ) { return x.so > y.so; } );

  // fuse neighbours that are contiguous in both tensors
  std::vector< D > l_fused;
  for( D const & l_d : l_dims ) {
    if( !l_fused.empty() ) {
      D & l_prev = l_fused.back();
      // l_prev is outer, l_d is inner
      if(    l_prev.so == l_d.so * l_d.size
          && l_prev.si == l_d.si * l_d.size ) {
        l_prev.size *= l_d.size;
        l_prev.so = l_d.so;
        l_prev.si = l_d.si;
        continue;
      }
    }
    l_fused.push_back( l_d );
  }
  if( (int64_t) l_fused.size() > kPermMaxDims ) {
    return fail( ETIR_COMPILATION_FAILED, "permute: too many non-fusable dimensions" );
  }
  plan.num_dims = (int32_t) l_fused.size();
  for( std::size_t l_di = 0; l_di < l_fused.size(); l_di++ ) {
    plan.size[l_di]  = l_fused[l_di].size;
    plan.s_in[l_di]  = l_fused[l_di].si;
    plan.s_out[l_di] = l_fused[l_di].so;
  }

  PermArgs & a = plan.args;
  a = PermArgs();
  a.num_elements = l_num;
  a.add = ( ktype == ETIR_KTYPE_ADD );

  int l_n = plan.num_dims;
  int l_dim_i = -1;  // unit stride in input
  int l_dim_o = -1;  // unit stride in output
  for( int l_di = 0; l_di < l_n; l_di++ ) {
    if( plan.s_in[l_di]  == 1 && l_dim_i < 0 ) l_dim_i = l_di;
    if( plan.s_out[l_di] == 1 && l_dim_o < 0 ) l_dim_o = l_di;
  }

  auto all_div = [&]( int64_t v, int skip0, int skip1 ) {
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if( l_di == skip0 || l_di == skip1 ) continue;
      if( plan.s_in[l_di] % v != 0 || plan.s_out[l_di] % v != 0 ) return false;
    }
    return true;
  };
  auto all_div4 = [&]( int skip0, int skip1 ) { return all_div( 4, skip0, skip1 ); };
  // 2-byte transpose with 16-byte reads: input rows in groups of 8 elements,
  // output rows in groups of 4, every other stride a multiple of those
  auto v16_ok = [&]( int di, int dof ) {
    if(    plan.elem_bytes != 2 || plan.size[di] % 8 != 0 || plan.s_in[dof] % 8 != 0 || plan.size[dof] % 4 != 0
        || plan.s_out[di] % 4 != 0 ) {
      return false;
    }
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if( l_di != di && plan.s_in[l_di] % 8 != 0 ) return false;
      if( l_di != dof && plan.s_out[l_di] % 4 != 0 ) return false;
    }
    return true;
  };
  // the output dim that continues the output's run after dim dof (output
  // stride = dof's size), not the input's unit-stride dim di; -1 if none
  auto fold_dim = [&]( int di, int dof ) {
    int l_f = -1;
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if(    l_di != di && l_di != dof && plan.s_out[l_di] == plan.size[dof]
          && plan.size[dof] * plan.size[l_di] < ( int64_t( 1 ) << 26 ) ) {
        l_f = l_di;
      }
    }
    return l_f;
  };

  if( ktype == ETIR_KTYPE_ZERO ) {
    plan.mode = PermMode::FILL;
    a.num_batch = l_n;
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      a.batch_size[l_di] = plan.size[l_di];
      a.batch_s_in[l_di] = 0;
      a.batch_s_out[l_di] = plan.s_out[l_di];
    }
    a.vec_ok = ( l_n > 0 && l_dim_o == l_n - 1 && plan.size[l_n-1] % 4 == 0 );
    for( int l_di = 0; l_di < l_n - 1 && a.vec_ok; l_di++ ) {
      if( plan.s_out[l_di] % 4 != 0 ) a.vec_ok = 0;
    }
    a.vec_wide = ( a.vec_ok && plan.elem_bytes == 2 && plan.size[l_n-1] % 8 == 0 );
    for( int l_di = 0; l_di < l_n - 1 && a.vec_wide; l_di++ ) {
      if( plan.s_out[l_di] % 8 != 0 ) a.vec_wide = 0;
    }
    return ETIR_SUCCESS;
  }

  // REG4 block side and its dim-length limits, in elements: a block row is
  // one vector -- 16 bytes for fp32 (4 x 4) and for bf16 when both unit dims
  // are multiples of 8 (8 x 8; else 4 x 4 with 8-byte rows), 32 bytes for
  // fp64 (4 x 4) -- and the limits measured for fp32 (a short dim up to 16,
  // both up to 32) scale with the elements per 4 bytes
  int64_t const l_vb = (    plan.elem_bytes == 2 && l_dim_i >= 0 && l_dim_o >= 0
                         && plan.size[l_dim_i] % 8 == 0 && plan.size[l_dim_o] % 8 == 0 ) ? 8 : 4;
  int64_t const l_scale = plan.elem_bytes == 2 ? 2 : 1;
  // 2-byte elements whose output unit-stride dim (above 16) the 16-byte
  // transpose can fold with the output's next dim (below) take that
  // transpose rather than REG4 (bf16 abcd->dcba 32,32,128,128: 66.9 against
  // 70.0 % of HBM peak; 24,32,128,128: 25.8 against 71.5 %)
  // (an input unit-stride dim of at least a tile side: shorter ones take the
  // tiled kernel below when not REG4)
  bool const l_fold16 = plan.elem_bytes == 2 && l_dim_i >= 0 && l_dim_o >= 0 && l_dim_i != l_dim_o
                     && plan.size[l_dim_i] >= kTile && plan.size[l_dim_o] > kReg4MaxShort
                     && v16_ok( l_dim_i, l_dim_o )
                     && fold_dim( l_dim_i, l_dim_o ) >= 0;
  int64_t const l_short = l_fold16 ? kReg4MaxShort : kReg4MaxShort * l_scale;
  int64_t const l_both = 32 * l_scale;

  // a long input unit-stride dim with a short output one: split it into an
  // inner part that, with the output's dim, fills one wave of blocks and an
  // outer part (the REG4 tiles below take the inner part whole)
  if(    l_dim_i >= 0 && l_dim_o >= 0 && l_dim_i != l_dim_o && l_n < kPermMaxDims
      && plan.size[l_dim_o] % l_vb == 0 && plan.size[l_dim_o] <= l_short
      && ( plan.size[l_dim_i] / l_vb ) * ( plan.size[l_dim_o] / l_vb ) > 64 ) {
    int64_t const l_lo = l_vb * ( 64 / ( plan.size[l_dim_o] / l_vb ) );
    if( plan.size[l_dim_i] % l_lo == 0 ) {
      for( int l_di = l_n; l_di > l_dim_i; l_di-- ) {
        plan.size[l_di]  = plan.size[l_di - 1];
        plan.s_in[l_di]  = plan.s_in[l_di - 1];
        plan.s_out[l_di] = plan.s_out[l_di - 1];
      }
      // dims stay in output order: the outer part has the larger output stride
      plan.size[l_dim_i]      = plan.size[l_dim_i + 1] / l_lo;
      plan.s_in[l_dim_i]      = l_lo;
      plan.s_out[l_dim_i]     = plan.s_out[l_dim_i + 1] * l_lo;
      plan.size[l_dim_i + 1]  = l_lo;
      if( l_dim_o > l_dim_i ) l_dim_o++;
      l_dim_i++;
      l_n++;
      plan.num_dims = l_n;
    }
  }

  if(    l_dim_i >= 0 && l_dim_o >= 0 && l_dim_i != l_dim_o
      && plan.size[l_dim_i] % l_vb == 0 && plan.size[l_dim_o] % l_vb == 0
      && (    std::min( plan.size[l_dim_i], plan.size[l_dim_o] ) <= l_short
           || (    std::max( plan.size[l_dim_i], plan.size[l_dim_o] ) <= l_both
                && ( plan.size[l_dim_i] * plan.elem_bytes ) % 128 == 0
                && ( plan.size[l_dim_o] * plan.elem_bytes ) % 128 == 0 ) )
      && ( plan.size[l_dim_i] / l_vb ) * ( plan.size[l_dim_o] / l_vb ) <= kThreads ) {
    // a short unit-stride dim: register-transposed blocks.  The dim that
    // continues the input's run (input stride size_i), else the output's,
    // else the largest other dim, is walked by consecutive lanes after i
    plan.mode = PermMode::REG4;
    plan.reg4_vb = (int32_t) l_vb;
    a.size_i  = plan.size[l_dim_i];
    a.size_o  = plan.size[l_dim_o];
    a.s_in_o  = plan.s_in[l_dim_o];
    a.s_out_i = plan.s_out[l_dim_i];
    auto other = [&]( int d ) { return d != l_dim_i && d != l_dim_o; };
    int l_dc = -1;
    for( int l_di = 0; l_di < l_n && l_dc < 0; l_di++ ) {
      if( other( l_di ) && plan.s_in[l_di] == a.size_i ) l_dc = l_di;
    }
    for( int l_di = 0; l_di < l_n && l_dc < 0; l_di++ ) {
      if( other( l_di ) && plan.s_out[l_di] == a.size_o ) l_dc = l_di;
    }
    if( l_dc < 0 ) {
      for( int l_di = 0; l_di < l_n; l_di++ ) {
        if( other( l_di ) && ( l_dc < 0 || plan.size[l_di] > plan.size[l_dc] ) ) l_dc = l_di;
      }
    }
    a.c_size  = l_dc >= 0 ? plan.size[l_dc] : 1;
    a.c_s_in  = l_dc >= 0 ? plan.s_in[l_dc] : 0;
    a.c_s_out = l_dc >= 0 ? plan.s_out[l_dc] : 0;
    // a workgroup's tile: all of i and o, c_chunk values of c -- one value
    // per thread group of (i/4 x o/4) threads, in the smallest workgroup of
    // 64, 128 or 256 threads that holds one value's blocks: small workgroups
    // measured faster than large ones on every 4-D shape (16,256,256,16 fp32:
    // 74 % of HBM peak at 64 threads, 62 % at 256, 54 % at 512).  Planner
    // options: ETIR_PERM_REG4_THREADS (64 ... 512) and ETIR_PERM_REG4_CPT, two
    // or four passes of 256 threads over c (longer runs of (c, i), measured
    // slower too)
    int64_t const l_blocks_c = ( a.size_i / l_vb ) * ( a.size_o / l_vb );
    int32_t const l_threads_small = l_blocks_c <= 64 ? 64 : ( l_blocks_c <= 128 ? 128 : kThreads );
    plan.reg4_threads = l_threads_small;
    // 2-byte elements with a 16-wide output run and an input run of 64 or
    // more: 512-thread workgroups (eight times the c values per workgroup)
    // measured faster on every such shape (bf16 acdb 128x16x64x128: 61 -> 76
    // % of HBM peak; five more, i of 64 to 256: 60-62 -> 74-77 %); an output
    // run of 8 or 32, a short input run, and fp32 gain nothing or lose
    if( plan.elem_bytes == 2 && a.size_o == 16 && a.size_i >= 64 && l_blocks_c <= 512 ) plan.reg4_threads = 512;
    plan.reg4_cpt = 1;
    if( char const * l_env = std::getenv( "ETIR_PERM_REG4_THREADS" ) ) {
      int const l_t = std::atoi( l_env );
      if( ( l_t == 512 || l_t == 256 || l_t == 128 || l_t == 64 ) && l_t >= l_blocks_c ) plan.reg4_threads = l_t;
    }
    if( char const * l_env = std::getenv( "ETIR_PERM_REG4_CPT" ) ) {
      int const l_v = std::atoi( l_env );
      if( l_v == 2 || l_v == 4 ) {
        plan.reg4_cpt = l_v;
        plan.reg4_threads = kThreads;
      }
    }
    a.c_chunk = (int32_t) std::max< int64_t >( 1, plan.reg4_threads / l_blocks_c );
    // stores straight from registers when the output run that one row of
    // blocks covers (o, continued by the chunk of c when c continues the
    // output's run) is whole 128-byte lines and both unit dims are at most
    // 16 (fp32 16,256,256,16: 77 % of HBM peak against 74 % through LDS; at
    // 32 x 32 the lanes of one store instruction spread over eight rows and
    // the LDS exchange is faster, 74 % against 65 %)
    int64_t const l_direct_run = a.size_o * plan.elem_bytes
                               * ( ( l_dc >= 0 && plan.s_out[l_dc] == a.size_o ) ? a.c_chunk : 1 );
    plan.reg4_direct = ( l_direct_run % 128 == 0 && plan.reg4_cpt == 1
                         && std::max( a.size_i, a.size_o ) <= 16 * l_scale );
    if( char const * l_env = std::getenv( "ETIR_PERM_REG4_DIRECT" ) ) {
      plan.reg4_direct = plan.reg4_direct && std::atoi( l_env ) != 0;
    }
    a.c_chunk *= plan.reg4_cpt;
    // LDS slot pitches: simulate both phases' 16-byte accesses (eight lanes
    // per LDS cycle, a slot covers 4 of the 64 four-byte banks; fp64's
    // 32-byte slots are counted as 16-byte ones) and take the padding with
    // the fewest conflicts among those whose tile fits the 64 KiB a
    // workgroup gets; where none does (several passes over c with a long i
    // run: bf16 acdb with a 128-wide input run, four passes, about 130 KiB)
    // the planner takes one pass of the smallest workgroup
    auto pick_slots = [&]() -> bool {
      int32_t const l_nig = int32_t( a.size_i / l_vb ), l_nog = int32_t( a.size_o / l_vb );
      int32_t const l_si = int32_t( a.size_i );
      int32_t const l_cw = a.c_chunk / plan.reg4_cpt, l_ct = a.c_chunk;
      int32_t const l_used = l_nig * l_nog * l_cw;
      bool const l_c_inner = a.c_s_out < a.s_out_i;
      int64_t l_best = -1;
      for( int32_t l_padi = 0; l_padi < 4; l_padi++ ) {
        for( int32_t l_padc = 0; l_padc < 16; l_padc++ ) {
          int32_t const l_pi = l_nog + l_padi, l_pc = l_si * l_pi + l_padc;
          if( int64_t( a.c_chunk ) * l_pc * l_vb * plan.elem_bytes > 65536 ) continue;
          int64_t l_cost = 0;
          auto group_cost = [&]( std::vector< int32_t > const & slots ) {
            for( std::size_t l_g = 0; l_g < slots.size(); l_g += 8 ) {
              int l_cnt[16] = { 0 };
              int l_mx = 0;
              for( std::size_t l_k = l_g; l_k < std::min( slots.size(), l_g + 8 ); l_k++ ) {
                l_mx = std::max( l_mx, ++l_cnt[slots[l_k] % 16] );
              }
              l_cost += l_mx;
            }
          };
          // phase 1: one instruction per (pass, q), lanes = threads
          for( int l_u = 0; l_u < plan.reg4_cpt; l_u++ ) {
            for( int l_q = 0; l_q < l_vb; l_q++ ) {
              std::vector< int32_t > l_sl;
              for( int32_t l_t = 0; l_t < l_used; l_t++ ) {
                int32_t const l_ig = l_t % l_nig, l_cl = ( l_t / l_nig ) % l_cw, l_og = l_t / l_nig / l_cw;
                l_sl.push_back( ( l_cl + l_u * l_cw ) * l_pc + ( int32_t( l_vb ) * l_ig + l_q ) * l_pi + l_og );
              }
              group_cost( l_sl );
            }
          }
          // phase 2: slots in output order
          std::vector< int32_t > l_sl;
          for( int32_t l_s = 0; l_s < l_si * l_ct * l_nog; l_s++ ) {
            int32_t const l_og = l_s % l_nog, l_s2 = l_s / l_nog;
            int32_t const l_cl = l_c_inner ? l_s2 % l_ct : l_s2 / l_si;
            int32_t const l_i  = l_c_inner ? l_s2 / l_ct : l_s2 % l_si;
            l_sl.push_back( l_cl * l_pc + l_i * l_pi + l_og );
          }
          group_cost( l_sl );
          if( l_best < 0 || l_cost < l_best ) {
            l_best = l_cost;
            a.slot_pi = l_pi;
            a.slot_pc = l_pc;
          }
        }
      }
      return l_best >= 0;
    };
    if( !pick_slots() ) {
      plan.reg4_cpt = 1;
      plan.reg4_threads = l_threads_small;
      plan.reg4_direct = false;
      a.c_chunk = (int32_t) std::max< int64_t >( 1, plan.reg4_threads / l_blocks_c );
      if( !pick_slots() ) return fail( ETIR_COMPILATION_FAILED, "permute: REG4 tile does not fit LDS" );
    }
    a.num_batch = 0;
    a.num_batch_total = 1;
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if( l_di == l_dim_i || l_di == l_dim_o || l_di == l_dc ) continue;
      a.batch_size[a.num_batch]  = plan.size[l_di];
      a.batch_s_in[a.num_batch]  = plan.s_in[l_di];
      a.batch_s_out[a.num_batch] = plan.s_out[l_di];
      a.num_batch_total *= plan.size[l_di];
      a.num_batch++;
    }
    // block rows as vectors: every stride a multiple of the row length
    a.vec_ok = ( a.s_in_o % l_vb == 0 && a.s_out_i % l_vb == 0 && all_div( l_vb, l_dim_i, l_dim_o ) ) ? 1 : 0;
    return ETIR_SUCCESS;
  }

  if( l_dim_i >= 0 && l_dim_i == l_dim_o && l_n > 2 && plan_rows( plan, l_dim_i ) ) {
    // a shared unit-stride dim of short rows: whole rows through LDS, no
    // tables (abcd->cabd 48,36,512,36: xx against yy TB/s tiled)
    return ETIR_SUCCESS;
  }

  if(    l_dim_i >= 0 && l_dim_o >= 0 && l_n > 1
      && (    ( plan.size[l_dim_i] < kTile && plan.size[l_dim_o] < kTile )
           || std::min( plan.size[l_dim_i], plan.size[l_dim_o] ) <= 8
           || plan.size[l_dim_i] <= 16 )
      && plan_tiled( plan, l_dim_i, l_dim_o ) ) {
    // both unit-stride dims shorter than a tile side, or one of them at most
    // 8 long (a 64 x 64 transpose tile would hold 8 of 64 rows: abc->cba at
    // 4,2048,2048 ran at 1.6 against 4.9 TB/s tiled), or the input's at most
    // 16 long (abcde->eabcd with e = 16: 3.6 against 4.2 TB/s); with one long
    // side and the other 16 or more (the output's) or 32 or more the
    // transpose is faster (5.1-6.3 against 4.6-5.3 TB/s); also when both are
    // the same short dim, where a plain vector copy reads or writes runs of
    // that dim's length only
    return ETIR_SUCCESS;
  }

  if( l_dim_i >= 0 && l_dim_o >= 0 && l_dim_i != l_dim_o ) {
    plan.mode = PermMode::TRANSPOSE;
    a.size_i  = plan.size[l_dim_i];
    a.size_o  = plan.size[l_dim_o];
    a.s_in_o  = plan.s_in[l_dim_o];
    a.s_out_i = plan.s_out[l_dim_i];
    // tile shape: the one whose padded tile grid wastes the least, 64 x 64
    // unless another fills at least 1.25 times as much of its tiles (fp32
    // dcba 32,32,128,128 on 128 x 32: 74 -> 76 % of HBM peak; dbca
    // 32,64,256,96 61.5 % against 53 %, 96,64,256,32 on 32 x 128 58 %
    // against 47 %)
    auto util = [&]( int64_t ti, int64_t to ) {
      return double( a.size_i ) / double( ( a.size_i + ti - 1 ) / ti * ti )
           * double( a.size_o ) / double( ( a.size_o + to - 1 ) / to * to );
    };
    plan.tr_shape = 0;
    double l_best = 1.25 * util( kTile, kTile );
    if( util( 128, 32 ) >= l_best ) { plan.tr_shape = 1; l_best = util( 128, 32 ); }
    if( util( 32, 128 ) > l_best )  plan.tr_shape = 2;
    int64_t l_ti = plan.tr_shape == 1 ? 128 : ( plan.tr_shape == 2 ? 32 : kTile );
    int64_t l_to = 4 * 4 * kThreads / l_ti;
    // 2-byte elements whose input rows allow 8-element vectors (and output
    // rows 4-element ones): the 16-byte-read transpose, 128 x 64 unless
    // 128 x 32 fills strictly more of its padded tile grid
    bool const l_v16 = v16_ok( l_dim_i, l_dim_o );
    // an output unit-stride dim that leaves 64-wide tiles part empty: the
    // output's next dim, if it continues the output's run, is folded into o
    // (not the input's unit dim: that one is i), and the tile is 128 x 64,
    // whose output rows are whole 128-byte lines (bf16 abcd->bdac
    // 36,48,36,512: 51.6 % of HBM peak on 128 x 32 tiles of o = c, 64.7 %
    // folded on 128 x 32, 71.0 % folded on 128 x 64)
    int const l_dim_o2 = ( l_v16 && a.size_o % 64 != 0 ) ? fold_dim( l_dim_i, l_dim_o ) : -1;
    a.o1_size = 0;
    if( l_dim_o2 >= 0 ) {
      a.o1_size  = int32_t( a.size_o );
      a.o1_magic = uint32_t( ( ( uint64_t( 1 ) << 32 ) + uint64_t( a.size_o ) - 1 ) / uint64_t( a.size_o ) );
      a.s_in_o2  = plan.s_in[l_dim_o2];
      a.size_o  *= plan.size[l_dim_o2];
    }
    if( l_v16 ) {
      plan.tr_shape = ( l_dim_o2 < 0 && util( 128, 32 ) > util( 128, 64 ) ) ? 4 : 3;
      l_ti = 128;
      l_to = ( plan.tr_shape == 3 ) ? 64 : 32;
    }
    a.tiles_i = ( a.size_i + l_ti - 1 ) / l_ti;
    a.tiles_o = ( a.size_o + l_to - 1 ) / l_to;
    a.num_batch = 0;
    a.num_batch_total = 1;
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if( l_di == l_dim_i || l_di == l_dim_o || l_di == l_dim_o2 ) continue;
      a.batch_size[a.num_batch]  = plan.size[l_di];
      a.batch_s_in[a.num_batch]  = plan.s_in[l_di];
      a.batch_s_out[a.num_batch] = plan.s_out[l_di];
      a.num_batch_total *= plan.size[l_di];
      a.num_batch++;
    }
    a.vec_ok = (    a.size_i % 4 == 0 && a.size_o % 4 == 0
                 && a.s_in_o % 4 == 0 && a.s_out_i % 4 == 0
                 && all_div4( l_dim_i, l_dim_o ) ) ? 1 : 0;
    a.nt_store = 1;
    return ETIR_SUCCESS;
  }

  // copy (same innermost dim) or gather
  a.num_batch = l_n;
  for( int l_di = 0; l_di < l_n; l_di++ ) {
    a.batch_size[l_di]  = plan.size[l_di];
    a.batch_s_in[l_di]  = plan.s_in[l_di];
    a.batch_s_out[l_di] = plan.s_out[l_di];
  }
  if(    l_n > 0 && l_dim_i == l_n - 1 && l_dim_o == l_n - 1
      && plan.size[l_n-1] % 4 == 0 && all_div4( l_n - 1, l_n - 1 ) ) {
    plan.mode = PermMode::COPY_VEC;
    a.vec_ok = 1;
    a.vec_wide = ( plan.elem_bytes == 2 && plan.size[l_n-1] % 8 == 0 && all_div( 8, l_n - 1, l_n - 1 ) ) ? 1 : 0;
  }
  else {
    plan.mode = PermMode::GATHER;
    a.vec_ok = 0;
  }
  return ETIR_SUCCESS;
}

int launch_permute( PermutePlan const & plan,
                    void const        * in,
                    void              * out,
                    hipStream_t         stream ) {
  if( plan.num_elements == 0 ) return ETIR_SUCCESS;
  if( out == nullptr || ( plan.mode != PermMode::FILL && in == nullptr ) ) {
    return fail( ETIR_NO_DATA_PTR_PROVIDED, "permute: null tensor pointer" );
  }
  PermArgs a = plan.args;
  a.in  = in;
  a.out = out;
  // the vector paths need their vectors aligned: 4 elements, REG4 one block
  // row (8 bf16 elements)
  uintptr_t const l_align = uintptr_t( ( plan.mode == PermMode::REG4 ? plan.reg4_vb
                                      : plan.mode == PermMode::ROWS ? plan.rows_vw : 4 ) * plan.elem_bytes );
  if( a.vec_ok ) {
    if(    ( uintptr_t( out ) % l_align ) != 0
        || ( plan.mode != PermMode::FILL && ( uintptr_t( in ) % l_align ) != 0 ) ) {
      a.vec_ok = 0;
    }
    // the 16-byte-read transpose reads 8 elements per vector
    if( plan.mode == PermMode::TRANSPOSE && plan.tr_shape >= 3 && uintptr_t( in ) % 16 != 0 ) a.vec_ok = 0;
  }
  if(    a.vec_wide
      && (    ( uintptr_t( out ) % 16 ) != 0
           || ( plan.mode != PermMode::FILL && ( uintptr_t( in ) % 16 ) != 0 ) ) ) {
    a.vec_wide = 0;
  }
  PermutePlan l_plan = plan;
  if( plan.mode == PermMode::COPY_VEC && !a.vec_ok ) l_plan.mode = PermMode::GATHER;
  if( plan.mode == PermMode::ROWS && !a.vec_ok && plan.rows_vw > 1 ) {
    // unaligned pointers: chunks of one element (same tile, same LDS bytes)
    l_plan.rows_vw = 1;
    a.rows_g     = int32_t( plan.rows_len );
    a.rows_pitch = int32_t( a.rows_ey * plan.rows_len );
  }

  if( plan.elem_bytes == 4 ) return launch_typed< float    >( l_plan, a, stream );
  if( plan.elem_bytes == 8 ) return launch_typed< double   >( l_plan, a, stream );
  if( plan.elem_bytes == 2 ) return launch_typed< uint16_t >( l_plan, a, stream );
  return fail( ETIR_INVALID_DTYPE, "permute: unsupported element size" );
}

}  // namespace etir
