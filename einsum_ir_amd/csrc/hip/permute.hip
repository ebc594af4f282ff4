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
//   - if both innermost dims coincide the copy is vectorised along them;
//   - anything else is a one-thread-per-element gather.
#include "etir_internal.h"
#include <algorithm>
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

constexpr int kTile = 64;
constexpr int kThreads = 256;

// LDS-tiled transpose of one 64x64 (i, o) tile per workgroup.
template< typename T >
__global__ __launch_bounds__( kThreads )
void perm_transpose_kernel( PermArgs a ) {
  __shared__ T l_tile[kTile][kTile + 1];

  int64_t l_bid = blockIdx.x;
  int64_t l_ti  = l_bid % a.tiles_i;  l_bid /= a.tiles_i;
  int64_t l_to  = l_bid % a.tiles_o;
  int64_t l_bb  = l_bid / a.tiles_o;

  int64_t l_off_in  = 0;
  int64_t l_off_out = 0;
  for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
    int64_t l_idx = l_bb % a.batch_size[l_d];
    l_bb /= a.batch_size[l_d];
    l_off_in  += l_idx * a.batch_s_in[l_d];
    l_off_out += l_idx * a.batch_s_out[l_d];
  }

  T const * l_in  = reinterpret_cast< T const * >( a.in )  + l_off_in;
  T       * l_out = reinterpret_cast< T       * >( a.out ) + l_off_out;

  int64_t const l_i0 = l_ti * kTile;
  int64_t const l_o0 = l_to * kTile;
  int const l_t  = threadIdx.x;
  int const l_c4 = l_t & 15;
  int const l_r  = l_t >> 4;

  // read: rows along o, 4 consecutive i per thread
#pragma unroll
  for( int l_p = 0; l_p < 4; l_p++ ) {
    int const l_row = l_r + 16 * l_p;
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
#pragma unroll
  for( int l_p = 0; l_p < 4; l_p++ ) {
    int const l_row = l_r + 16 * l_p;
    int64_t const l_i = l_i0 + l_row;
    int64_t const l_o = l_o0 + 4 * l_c4;
    T l_v[4];
#pragma unroll
    for( int l_e = 0; l_e < 4; l_e++ ) l_v[l_e] = l_tile[4 * l_c4 + l_e][l_row];

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
        *l_ptr = l_tmp;
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

// One thread per VW consecutive output elements of the innermost dim.
// Dims are (outer -> inner) in a.batch_*; for VW == 4 the innermost dim has
// unit stride in both tensors and a size divisible by 4.
template< typename T, int VW, bool FILL >
__global__ __launch_bounds__( kThreads )
void perm_gather_kernel( PermArgs a ) {
  int64_t const l_num_items = a.num_elements / VW;
  for( int64_t l_item = int64_t( blockIdx.x ) * kThreads + threadIdx.x;
       l_item < l_num_items;
       l_item += int64_t( gridDim.x ) * kThreads ) {
    int64_t l_rem = l_item * VW;
    int64_t l_off_in  = 0;
    int64_t l_off_out = 0;
    for( int l_d = a.num_batch - 1; l_d >= 0; l_d-- ) {
      int64_t l_sz  = a.batch_size[l_d];
      int64_t l_idx = l_rem % l_sz;
      l_rem /= l_sz;
      l_off_in  += l_idx * a.batch_s_in[l_d];
      l_off_out += l_idx * a.batch_s_out[l_d];
    }
    T * l_out = reinterpret_cast< T * >( a.out ) + l_off_out;
    if( FILL ) {
      if( VW == 4 ) {
        Vec4< T > l_z;
#pragma unroll
        for( int l_e = 0; l_e < 4; l_e++ ) l_z.v[l_e] = T(0);
        *reinterpret_cast< Vec4< T > * >( l_out ) = l_z;
      }
      else {
        *l_out = T(0);
      }
      continue;
    }
    T const * l_in = reinterpret_cast< T const * >( a.in ) + l_off_in;
    if( VW == 4 ) {
      Vec4< T > l_v = *reinterpret_cast< Vec4< T > const * >( l_in );
      if( a.add ) {
        Vec4< T > l_old = *reinterpret_cast< Vec4< T > * >( l_out );
#pragma unroll
        for( int l_e = 0; l_e < 4; l_e++ ) l_v.v[l_e] = Elem< T >::add( l_old.v[l_e], l_v.v[l_e] );
      }
      *reinterpret_cast< Vec4< T > * >( l_out ) = l_v;
    }
    else {
      T l_v = *l_in;
      *l_out = a.add ? Elem< T >::add( *l_out, l_v ) : l_v;
    }
  }
}

template< typename T >
int launch_typed( PermutePlan const & p,
                  PermArgs          & a,
                  hipStream_t         stream ) {
  if( p.mode == PermMode::TRANSPOSE ) {
    int64_t l_blocks = a.tiles_i * a.tiles_o * a.num_batch_total;
    if( l_blocks > 0x7fffffffLL ) {
      return fail( ETIR_UNDEFINED_ERROR, "permute: grid too large" );
    }
    hipLaunchKernelGGL( perm_transpose_kernel< T >, dim3( (uint32_t) l_blocks ), dim3( kThreads ), 0, stream, a );
  }
  else {
    int const l_vw = ( p.mode == PermMode::COPY_VEC || ( p.mode == PermMode::FILL && a.vec_ok ) ) && a.vec_ok ? 4 : 1;
    int64_t l_items = a.num_elements / l_vw;
    int64_t l_blocks = ( l_items + kThreads - 1 ) / kThreads;
    l_blocks = std::min< int64_t >( l_blocks, 65536 );
    if( l_blocks < 1 ) l_blocks = 1;
    bool const l_fill = ( p.mode == PermMode::FILL );
    if( l_fill ) {
      if( l_vw == 4 ) hipLaunchKernelGGL( ( perm_gather_kernel< T, 4, true > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), 0, stream, a );
      else            hipLaunchKernelGGL( ( perm_gather_kernel< T, 1, true > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), 0, stream, a );
    }
    else {
      if( l_vw == 4 ) hipLaunchKernelGGL( ( perm_gather_kernel< T, 4, false > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), 0, stream, a );
      else            hipLaunchKernelGGL( ( perm_gather_kernel< T, 1, false > ), dim3( (uint32_t) l_blocks ), dim3( kThreads ), 0, stream, a );
    }
  }
  hipError_t l_err = hipGetLastError();
  if( l_err != hipSuccess ) {
    return fail( ETIR_UNDEFINED_ERROR, std::string( "permute launch failed: " ) + hipGetErrorString( l_err ) );
  }
  return ETIR_SUCCESS;
}

}  // namespace

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

  auto all_div4 = [&]( int skip0, int skip1 ) {
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if( l_di == skip0 || l_di == skip1 ) continue;
      if( plan.s_in[l_di] % 4 != 0 || plan.s_out[l_di] % 4 != 0 ) return false;
    }
    return true;
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
    return ETIR_SUCCESS;
  }

  if( l_dim_i >= 0 && l_dim_o >= 0 && l_dim_i != l_dim_o ) {
    plan.mode = PermMode::TRANSPOSE;
    a.size_i  = plan.size[l_dim_i];
    a.size_o  = plan.size[l_dim_o];
    a.s_in_o  = plan.s_in[l_dim_o];
    a.s_out_i = plan.s_out[l_dim_i];
    a.tiles_i = ( a.size_i + kTile - 1 ) / kTile;
    a.tiles_o = ( a.size_o + kTile - 1 ) / kTile;
    a.num_batch = 0;
    a.num_batch_total = 1;
    for( int l_di = 0; l_di < l_n; l_di++ ) {
      if( l_di == l_dim_i || l_di == l_dim_o ) continue;
      a.batch_size[a.num_batch]  = plan.size[l_di];
      a.batch_s_in[a.num_batch]  = plan.s_in[l_di];
      a.batch_s_out[a.num_batch] = plan.s_out[l_di];
      a.num_batch_total *= plan.size[l_di];
      a.num_batch++;
    }
    a.vec_ok = (    a.size_i % 4 == 0 && a.size_o % 4 == 0
                 && a.s_in_o % 4 == 0 && a.s_out_i % 4 == 0
                 && all_div4( l_dim_i, l_dim_o ) ) ? 1 : 0;
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
  // 16-byte alignment (4 elements) is required for the vector paths
  uintptr_t const l_align = uintptr_t( 4 * plan.elem_bytes );
  if( a.vec_ok ) {
    if(    ( uintptr_t( out ) % l_align ) != 0
        || ( plan.mode != PermMode::FILL && ( uintptr_t( in ) % l_align ) != 0 ) ) {
      a.vec_ok = 0;
    }
  }
  PermutePlan l_plan = plan;
  if( plan.mode == PermMode::COPY_VEC && !a.vec_ok ) l_plan.mode = PermMode::GATHER;

  if( plan.elem_bytes == 4 ) return launch_typed< float    >( l_plan, a, stream );
  if( plan.elem_bytes == 8 ) return launch_typed< double   >( l_plan, a, stream );
  if( plan.elem_bytes == 2 ) return launch_typed< uint16_t >( l_plan, a, stream );
  return fail( ETIR_INVALID_DTYPE, "permute: unsupported element size" );
}

}  // namespace etir
