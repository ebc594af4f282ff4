// Contraction planner: loop IR -> one kernel launch.
//
// Replaces the reference's loop-nest lowering and primitive choice
//   BinaryContractionTpp::compile        reference src/backend/BinaryContractionTpp.cpp:4-127
//   ContractionOptimizer::optimize       reference src/basic/binary/ContractionOptimizer.cpp:47-74
//     (sort_and_fuse_iters :76-111, set_primitive_iters :232-584,
//      reorder_and_parallelize_iters :586-679)
//   ContractionBackend::set_kernel_shape reference src/basic/binary/ContractionBackend.cpp:518-678
//
// The reference picks a libxsmm GEMM/BRGEMM over the innermost unit-stride
// loops and runs every other loop on the host.  Here all loops of one type are
// flattened into a single kernel index (C -> grid batch, M -> MFMA rows,
// N -> MFMA columns, K -> reduction) and described by offset tables, so the
// whole contraction is one launch:
//   1. size-1 loops are dropped (ContractionOptimizer::remove_empty_iters, :113-121);
//   2. the kernel's column index (lanes 0..31 of a wave) is put on the
//      output's unit-stride type, swapping the roles of left and right when
//      the output is M-contiguous, so that epilogue stores coalesce;
//   3. inside each type the loops are ordered so that the operand's
//      unit-stride loop is innermost (the analogue of choosing the
//      primitive's unit-stride m/k loops); kernel rows the A operand is not
//      contiguous along follow the output's order instead;
//   4. the tables are enumerated and inspected: runs of consecutive offsets
//      select 16-byte vector loads along M/N or along K; a single-loop K index
//      becomes an affine offset (no table reads in the K loop);
//   5. the tile shape is chosen from dtype and the number of output tiles.
#include "etir_internal.h"
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <sstream>

namespace etir {

int launch_contract_tile( int32_t tile, int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                          uint32_t grid, hipStream_t stream );
int launch_contract_f64_64x64( int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                               uint32_t grid, hipStream_t stream );
int launch_contract_cpx( bool f64, int32_t ma, int32_t mb, bool kaff, ContractArgs const & a,
                         uint32_t grid, hipStream_t stream );
int launch_contract_bf16_dma( int32_t ma, int32_t mb, int32_t variant, ContractArgs const & a,
                              uint32_t grid, hipStream_t stream );
int launch_contract_panel( ContractArgs const & a, hipStream_t stream );
int launch_contract_kwave( int32_t waves, int32_t kw, ContractArgs const & a, uint32_t grid,
                           hipStream_t stream );
int launch_contract_f32_dma( int32_t ma, int32_t mb, ContractArgs const & a, uint32_t grid, hipStream_t stream );
int launch_contract_gemv( bool bf16_in, ContractArgs const & a, hipStream_t stream );
int launch_contract_skinny( bool bf16_in, ContractArgs const & a, hipStream_t stream );

namespace {

// tensor slots inside a loop
enum { T_L = 0, T_R = 1, T_AUX = 2, T_OUT = 3 };

struct Loop {
  int32_t type;
  int64_t size;
  int64_t s[4];
};

// enumerates sum_d digit_d * stride_d over the mixed-radix index of dims
// (outer -> inner)
std::vector< int64_t > enumerate( std::vector< Loop > const & dims, int slot ) {
  int64_t l_total = 1;
  for( Loop const & l_d : dims ) l_total *= l_d.size;
  std::vector< int64_t > l_tab( (std::size_t) l_total, 0 );
  if( l_total == 0 ) return l_tab;
  // fill from the innermost dim outwards: after processing a dim the first
  // l_filled entries hold the offsets of all inner digits
  int64_t l_filled = 1;
  for( int64_t l_di = (int64_t) dims.size() - 1; l_di >= 0; l_di-- ) {
    int64_t const l_sz = dims[l_di].size;
    int64_t const l_st = dims[l_di].s[slot];
    for( int64_t l_it = 1; l_it < l_sz; l_it++ ) {
      for( int64_t l_e = 0; l_e < l_filled; l_e++ ) {
        l_tab[l_it * l_filled + l_e] = l_tab[l_e] + l_it * l_st;
      }
    }
    l_filled *= l_sz;
  }
  return l_tab;
}

// true if tab is made of aligned runs of length v with unit increments and
// every run starts at a multiple of align
bool runs_contiguous( std::vector< int64_t > const & tab, int64_t v, int64_t align ) {
  if( (int64_t) tab.size() % v != 0 ) return false;
  for( std::size_t l_g = 0; l_g < tab.size(); l_g += v ) {
    if( tab[l_g] % align != 0 ) return false;
    for( int64_t l_e = 1; l_e < v; l_e++ ) {
      if( tab[l_g + l_e] != tab[l_g] + l_e ) return false;
    }
  }
  return true;
}

bool all_multiple( std::vector< int64_t > const & tab, int64_t align ) {
  for( int64_t l_v : tab ) if( l_v % align != 0 ) return false;
  return true;
}

bool fits_i32( std::vector< int64_t > const & tab ) {
  for( int64_t l_v : tab ) {
    if( l_v < 0 || l_v > std::numeric_limits< int32_t >::max() ) return false;
  }
  return true;
}

// sorts dims by their stride in `slot`, largest stride (outermost) first
void order_dims( std::vector< Loop > & dims, int slot ) {
  std::stable_sort( dims.begin(), dims.end(),
                    [slot]( Loop const & x, Loop const & y ) { return x.s[slot] > y.s[slot]; } );
}

// moves the first dim whose stride in `slot` is 1 to the innermost position;
// returns true if such a dim exists
bool unit_innermost( std::vector< Loop > & dims, int slot ) {
  for( std::size_t l_i = 0; l_i < dims.size(); l_i++ ) {
    if( dims[l_i].s[slot] == 1 ) {
      Loop l_d = dims[l_i];
      dims.erase( dims.begin() + l_i );
      dims.push_back( l_d );
      return true;
    }
  }
  return false;
}

std::string dims_str( std::vector< Loop > const & dims ) {
  std::ostringstream l_s;
  l_s << "[";
  for( std::size_t l_i = 0; l_i < dims.size(); l_i++ ) {
    if( l_i ) l_s << ",";
    l_s << dims[l_i].size;
  }
  l_s << "]";
  return l_s.str();
}

char const * mode_str( int32_t m ) {
  if( m == LOAD_VEC_MN ) return "vec_mn";
  if( m == LOAD_VEC_K )  return "vec_k";
  if( m == LOAD_VEC8_MN ) return "vec8_mn";
  if( m == LOAD_VEC8_K )  return "vec8_k";
  return "scalar";
}

char const * tile_str( int32_t t ) {
  switch( t ) {
    case TILE_F32_128x128:  return "f32_128x128x32";
    case TILE_F32_64x64:    return "f32_64x64x32";
    case TILE_BF16_256x256: return "bf16_256x256x64";
    case TILE_BF16_256x128: return "bf16_256x128x32";
    case TILE_BF16_DMA_256x256: return "bf16_dma_256x256";
    case TILE_BF16_DMA_256x128: return "bf16_dma_256x128";
    case TILE_BF16_128x128: return "bf16_128x128x64";
    case TILE_BF16_64x64:   return "bf16_64x64x64";
    case TILE_F64_64x64:    return "f64_64x64x16";
    case TILE_CPX_F32_64x64: return "cpx_f32_64x64x16";
    case TILE_CPX_F64_64x64: return "cpx_f64_64x64x16";
    case TILE_F32_KWAVE_32x32: return "f32_kwave_32x32";
    case TILE_F32_DMA_128x128: return "f32_dma_128x128x32";
    case TILE_GEMV:            return "gemv";
    case TILE_SKINNY:          return "skinny";
    case TILE_PANEL:           return "panel";
    default:                return "?";
  }
}

void tile_shape( int32_t t, int64_t & bm, int64_t & bn ) {
  switch( t ) {
    case TILE_F32_128x128:  bm = 128; bn = 128; break;
    case TILE_F32_64x64:    bm = 64;  bn = 64;  break;
    case TILE_BF16_256x256: bm = 256; bn = 256; break;
    case TILE_BF16_256x128: bm = 256; bn = 128; break;
    case TILE_BF16_DMA_256x256: bm = 256; bn = 256; break;
    case TILE_BF16_DMA_256x128: bm = 256; bn = 128; break;
    case TILE_F32_KWAVE_32x32: bm = 32; bn = 32; break;
    case TILE_BF16_128x128: bm = 128; bn = 128; break;
    case TILE_F32_DMA_128x128: bm = 128; bn = 128; break;
    default:                bm = 64;  bn = 64;  break;
  }
}

}  // namespace

namespace {

// next 256-byte aligned piece of the caller's region, or a clear error
int place_take( DevicePlacement & place, std::size_t bytes, void ** out, char const * what ) {
  std::size_t const l_start = ( place.used + 255 ) & ~std::size_t( 255 );
  if( l_start + bytes > place.capacity ) {
    return fail( ETIR_UNDEFINED_ERROR, std::string( "contraction: the " ) + what + " need "
                                        + std::to_string( l_start + bytes ) + " bytes of scratch, more than the "
                                        + std::to_string( place.capacity ) + " the allocation-free entry point has" );
  }
  *out = place.base + l_start;
  place.used = l_start + bytes;
  return ETIR_SUCCESS;
}

int plan_contraction_impl( int64_t            num_loops,
                           int32_t const    * dim_types,
                           int64_t const    * sizes,
                           int64_t const    * strides_left,
                           int64_t const    * strides_right,
                           int64_t const    * strides_out_aux,
                           int64_t const    * strides_out,
                           int32_t            dtype_left,
                           int32_t            dtype_right,
                           int32_t            dtype_comp,
                           int32_t            dtype_out,
                           int32_t            ktype_first_touch,
                           int32_t            ktype_main,
                           int32_t            ktype_last_touch,
                           bool               allow_split,
                           ContractionPlan  & plan,
                           DevicePlacement  * place ) {
  plan = ContractionPlan();
  plan.placed = ( place != nullptr );

  // ---------------------------------------------------------------- checks
  bool const l_f32  = dtype_left == ETIR_FP32 && dtype_right == ETIR_FP32
                   && dtype_comp == ETIR_FP32 && dtype_out == ETIR_FP32;
  bool const l_bf16 = dtype_left == ETIR_BF16 && dtype_right == ETIR_BF16
                   && dtype_comp == ETIR_FP32
                   && ( dtype_out == ETIR_FP32 || dtype_out == ETIR_BF16 );
  bool const l_f64  = dtype_left == ETIR_FP64 && dtype_right == ETIR_FP64
                   && dtype_comp == ETIR_FP64 && dtype_out == ETIR_FP64;
  if( !l_f32 && !l_bf16 && !l_f64 ) {
    return fail( ETIR_INVALID_DTYPE, "contraction: unsupported dtype combination" );
  }
  // complex: CPX_MADD with the reference BLAS backend's touch kernels
  // (BinaryContractionBlas.cpp:68-80)
  bool const l_cpx = ( ktype_main == ETIR_KTYPE_CPX_MADD );
  if( l_cpx ) {
    if( l_bf16 ) return fail( ETIR_INVALID_DTYPE, "contraction: complex kernels take FP32 or FP64" );
    if(    ktype_first_touch != ETIR_KTYPE_ZERO && ktype_first_touch != ETIR_KTYPE_CPX_ZERO
        && ktype_first_touch != ETIR_KTYPE_UNDEFINED ) {
      return fail( ETIR_INVALID_KTYPE, "contraction: unsupported complex first-touch kernel" );
    }
    if( ktype_last_touch != ETIR_KTYPE_UNDEFINED ) {
      return fail( ETIR_INVALID_KTYPE, "contraction: complex contractions have no last-touch kernel" );
    }
  }
  else {
    if( ktype_main != ETIR_KTYPE_MADD ) {
      return fail( ETIR_INVALID_KTYPE, "contraction: main kernel must be MADD or CPX_MADD" );
    }
    if(    ktype_first_touch != ETIR_KTYPE_ZERO && ktype_first_touch != ETIR_KTYPE_COPY
        && ktype_first_touch != ETIR_KTYPE_ADD  && ktype_first_touch != ETIR_KTYPE_UNDEFINED ) {
      return fail( ETIR_COMPILATION_FAILED, "contraction: unsupported first-touch kernel" );
    }
    if(    ktype_last_touch != ETIR_KTYPE_RELU && ktype_last_touch != ETIR_KTYPE_ADD
        && ktype_last_touch != ETIR_KTYPE_UNDEFINED ) {
      return fail( ETIR_COMPILATION_FAILED, "contraction: unsupported last-touch kernel" );
    }
  }
  if( num_loops < 0 || ( num_loops > 0 && ( dim_types == nullptr || sizes == nullptr
                                            || strides_left == nullptr || strides_right == nullptr
                                            || strides_out == nullptr ) ) ) {
    return fail( ETIR_COMPILATION_FAILED, "contraction: invalid loop arrays" );
  }

  plan.dtype_in    = dtype_left;
  plan.dtype_comp  = dtype_comp;
  plan.dtype_out   = dtype_out;
  plan.first_touch = ktype_first_touch;
  plan.last_touch  = ktype_last_touch;
  plan.needs_aux   =    ktype_first_touch == ETIR_KTYPE_COPY
                     || ktype_first_touch == ETIR_KTYPE_ADD
                     || ktype_last_touch  == ETIR_KTYPE_ADD;
  // without explicit aux strides the aux tensor shares the output's layout
  // (reference src/backend/BinaryContractionTpp.cpp:36-41)
  int64_t const * l_s_aux = strides_out_aux != nullptr ? strides_out_aux : strides_out;

  // ------------------------------------------------------------- loop sets
  std::vector< Loop > l_c, l_m, l_n, l_k, l_x;
  for( int64_t l_lo = 0; l_lo < num_loops; l_lo++ ) {
    if( sizes[l_lo] < 0 ) return fail( ETIR_COMPILATION_FAILED, "contraction: negative loop size" );
    if(    strides_left[l_lo] < 0 || strides_right[l_lo] < 0 || strides_out[l_lo] < 0
        || l_s_aux[l_lo] < 0 ) {
      return fail( ETIR_COMPILATION_FAILED, "contraction: negative stride" );
    }
    Loop l_lp{ dim_types[l_lo], sizes[l_lo],
               { strides_left[l_lo], strides_right[l_lo], l_s_aux[l_lo], strides_out[l_lo] } };
    if( l_lp.type == ETIR_DIM_I || l_lp.type == ETIR_DIM_J ) continue;
    if( l_lp.type == ETIR_DIM_CPX ) {
      l_x.push_back( l_lp );
      continue;
    }
    if( l_lp.size == 1 ) continue;
    if(      l_lp.type == ETIR_DIM_C ) l_c.push_back( l_lp );
    else if( l_lp.type == ETIR_DIM_M ) l_m.push_back( l_lp );
    else if( l_lp.type == ETIR_DIM_N ) l_n.push_back( l_lp );
    else if( l_lp.type == ETIR_DIM_K ) l_k.push_back( l_lp );
    else return fail( ETIR_COMPILATION_FAILED, "contraction: invalid dimension type" );
  }

  if( l_cpx != ( l_x.size() > 0 ) ) {
    return fail( ETIR_INVALID_CPX_DIM, "contraction: CPX_MADD needs exactly one CPX loop and CPX loops need CPX_MADD" );
  }
  if( l_x.size() > 1 || ( l_cpx && l_x[0].size != 2 ) ) {
    return fail( ETIR_INVALID_CPX_DIM, "contraction: the complex loop must be unique and of size 2" );
  }
  auto prod = []( std::vector< Loop > const & d ) {
    int64_t l_p = 1;
    for( Loop const & l_x : d ) l_p *= l_x.size;
    return l_p;
  };
  int64_t const l_size_c = prod( l_c );
  int64_t const l_size_m = prod( l_m );
  int64_t const l_size_n = prod( l_n );
  int64_t const l_size_k = prod( l_k );

  // ------------------------------------------------------------ role swap
  // kernel columns (lane index) go to the output's unit-stride type
  bool l_swap = false;
  for( Loop const & l_x : l_m ) if( l_x.s[T_OUT] == 1 ) l_swap = true;
  plan.swapped = l_swap;

  // kernel operand slots: A (rows), B (columns)
  int const l_sa = l_swap ? T_R : T_L;
  int const l_sb = l_swap ? T_L : T_R;
  std::vector< Loop > l_km = l_swap ? l_n : l_m;   // kernel-M loops (A, aux, out)
  std::vector< Loop > l_kn = l_swap ? l_m : l_n;   // kernel-N loops (B, aux, out)
  int64_t const l_kern_m = l_swap ? l_size_n : l_size_m;
  int64_t const l_kern_n = l_swap ? l_size_m : l_size_n;

  int64_t const l_esz = ( dtype_left == ETIR_BF16 ) ? 2 : ( dtype_left == ETIR_FP64 ? 8 : 4 );
  int64_t const l_vk  = 16 / l_esz;   // elements per 16-byte vector

  // ordering: kernel rows follow A when A is read along them, otherwise the
  // output (neighbouring tile rows then sit close in memory for the stores)
  bool l_a_unit_m = false;
  for( Loop const & l_x : l_km ) if( l_x.s[l_sa] == 1 ) l_a_unit_m = true;
  order_dims( l_km, l_a_unit_m ? l_sa : T_OUT );
  if( l_a_unit_m ) unit_innermost( l_km, l_sa );
  order_dims( l_kn, T_OUT );
  if( !unit_innermost( l_kn, T_OUT ) ) unit_innermost( l_kn, l_sb );
  // K: the operand whose unit-stride loop is a K loop decides the order
  bool l_a_unit_k = false, l_b_unit_k = false;
  for( Loop const & l_x : l_k ) {
    if( l_x.s[l_sa] == 1 ) l_a_unit_k = true;
    if( l_x.s[l_sb] == 1 ) l_b_unit_k = true;
  }
  int const l_k_slot = l_a_unit_k ? l_sa : ( l_b_unit_k ? l_sb : l_sa );
  order_dims( l_k, l_k_slot );
  unit_innermost( l_k, l_k_slot );
  order_dims( l_c, T_OUT );

  // --------------------------------------------------------------- tables
  std::vector< int64_t > l_tc_a   = enumerate( l_c, l_sa );
  std::vector< int64_t > l_tc_b   = enumerate( l_c, l_sb );
  std::vector< int64_t > l_tc_aux = enumerate( l_c, T_AUX );
  std::vector< int64_t > l_tc_out = enumerate( l_c, T_OUT );
  std::vector< int64_t > l_tm_a   = enumerate( l_km, l_sa );
  std::vector< int64_t > l_tm_aux = enumerate( l_km, T_AUX );
  std::vector< int64_t > l_tm_out = enumerate( l_km, T_OUT );
  std::vector< int64_t > l_tn_b   = enumerate( l_kn, l_sb );
  std::vector< int64_t > l_tn_aux = enumerate( l_kn, T_AUX );
  std::vector< int64_t > l_tn_out = enumerate( l_kn, T_OUT );
  std::vector< int64_t > l_tk_a   = enumerate( l_k, l_sa );
  std::vector< int64_t > l_tk_b   = enumerate( l_k, l_sb );

  int64_t const l_max_i32 = std::numeric_limits< int32_t >::max();
  if(    l_size_m > l_max_i32 || l_size_n > l_max_i32 || l_size_k > l_max_i32
      || l_size_c > l_max_i32 ) {
    return fail( ETIR_COMPILATION_FAILED, "contraction: flattened index exceeds int32" );
  }
  if(    !fits_i32( l_tm_a ) || !fits_i32( l_tm_aux ) || !fits_i32( l_tm_out )
      || !fits_i32( l_tn_b ) || !fits_i32( l_tn_aux ) || !fits_i32( l_tn_out )
      || !fits_i32( l_tk_a ) || !fits_i32( l_tk_b ) ) {
    return fail( ETIR_COMPILATION_FAILED, "contraction: per-type offsets exceed int32" );
  }
  int64_t const l_total_entries = 4 * l_size_c + 3 * ( l_size_m + l_size_n ) + 2 * l_size_k;
  if( l_total_entries > ( int64_t( 1 ) << 27 ) ) {
    return fail( ETIR_COMPILATION_FAILED, "contraction: offset tables too large" );
  }

  // ------------------------------------------------------- load modes
  auto pick_mode = [&]( std::vector< int64_t > const & rows,
                        std::vector< int64_t > const & tk,
                        std::vector< int64_t > const & tc ) -> int32_t {
    // 16-byte vectors of consecutive rows (4 fp32 / 8 bf16)
    if(    rows.size() > 0 && runs_contiguous( rows, l_vk, l_vk )
        && all_multiple( tk, l_vk ) && all_multiple( tc, l_vk ) ) {
      return LOAD_VEC_MN;
    }
    // 16-byte vectors along K
    if(    tk.size() > 0 && runs_contiguous( tk, l_vk, l_vk )
        && all_multiple( rows, l_vk ) && all_multiple( tc, l_vk ) ) {
      return LOAD_VEC_K;
    }
    // fp32 runs of even length that are not multiples of 4 (odd mode sizes
    // times 2, as in the einsum_benchmark MERA network): 8-byte vectors on
    // the generic fp32 tiles
    if( l_f32 && !l_cpx ) {
      if(    rows.size() > 0 && runs_contiguous( rows, 2, 2 )
          && all_multiple( tk, 2 ) && all_multiple( tc, 2 ) ) {
        return LOAD_VEC8_MN;
      }
      if(    tk.size() > 0 && runs_contiguous( tk, 2, 2 )
          && all_multiple( rows, 2 ) && all_multiple( tc, 2 ) ) {
        return LOAD_VEC8_K;
      }
    }
    return LOAD_SCALAR;
  };
  plan.mode_a = pick_mode( l_tm_a, l_tk_a, l_tc_a );
  plan.mode_b = pick_mode( l_tn_b, l_tk_b, l_tc_b );
  // complex: the imaginary parts are loaded like the real ones from base +
  // cpx stride, so that offset has to keep the 16-byte vector alignment
  if( l_cpx && l_x[0].s[l_sa] % l_vk != 0 ) plan.mode_a = LOAD_SCALAR;
  if( l_cpx && l_x[0].s[l_sb] % l_vk != 0 ) plan.mode_b = LOAD_SCALAR;

  bool l_k_affine = true;
  int64_t l_sk_a = l_tk_a.size() > 1 ? l_tk_a[1] : 0;
  int64_t l_sk_b = l_tk_b.size() > 1 ? l_tk_b[1] : 0;
  for( std::size_t l_i = 0; l_i < l_tk_a.size(); l_i++ ) {
    if( l_tk_a[l_i] != int64_t( l_i ) * l_sk_a || l_tk_b[l_i] != int64_t( l_i ) * l_sk_b ) {
      l_k_affine = false;
      break;
    }
  }

  // ---------------------------------------------------------- tile choice
  auto n_tiles = [&]( int32_t t ) {
    int64_t l_bm, l_bn;
    tile_shape( t, l_bm, l_bn );
    return ( ( l_kern_m + l_bm - 1 ) / l_bm ) * ( ( l_kern_n + l_bn - 1 ) / l_bn ) * l_size_c;
  };
  int64_t const l_cus = 256;
  // useful fraction of the padded tile grid times the fraction of CUs with a
  // tile: M = 64 on 128 x 128 tiles wastes half of every tile
  auto score = [&]( int32_t t ) {
    int64_t l_bm, l_bn;
    tile_shape( t, l_bm, l_bn );
    double const l_pad = double( ( ( l_kern_m + l_bm - 1 ) / l_bm ) * l_bm )
                       * double( ( ( l_kern_n + l_bn - 1 ) / l_bn ) * l_bn );
    double const l_util = l_pad > 0.0 ? double( l_kern_m ) * double( l_kern_n ) / l_pad : 1.0;
    return l_util * std::min( 1.0, double( n_tiles( t ) ) / double( l_cus ) );
  };
  if( l_cpx ) {
    plan.tile = l_f64 ? TILE_CPX_F64_64x64 : TILE_CPX_F32_64x64;
  }
  else if( l_f64 ) {
    plan.tile = TILE_F64_64x64;
  }
  else if( l_f32 ) {
    // the larger tile unless the smaller one wastes clearly less
    plan.tile = ( score( TILE_F32_128x128 ) >= 0.95 * score( TILE_F32_64x64 ) ) ? TILE_F32_128x128 : TILE_F32_64x64;
  }
  else {
    if(      n_tiles( TILE_BF16_256x128 ) >= 2 * l_cus ) plan.tile = TILE_BF16_256x128;
    else if( n_tiles( TILE_BF16_128x128 ) >= l_cus ) plan.tile = TILE_BF16_128x128;
    else                                             plan.tile = TILE_BF16_64x64;
  }
  // direct-to-LDS kernel: 16-byte vector modes on both operands, affine K,
  // every byte offset below the buffer range (2^31), and enough 256 x 256
  // tiles to give each CU at least one
  auto max_of = []( std::vector< int64_t > const & t ) {
    int64_t l_m = 0;
    for( int64_t l_v : t ) l_m = std::max( l_m, l_v );
    return l_m;
  };
  bool const l_dma_ok =
         l_bf16
      && ( plan.mode_a == LOAD_VEC_MN || plan.mode_a == LOAD_VEC_K )
      && ( plan.mode_b == LOAD_VEC_MN || plan.mode_b == LOAD_VEC_K )
      && l_k_affine
      && 2 * ( max_of( l_tm_a ) + std::max< int64_t >( l_size_k - 1, 0 ) * l_sk_a ) + 64 < ( int64_t( 1 ) << 31 )
      && 2 * ( max_of( l_tn_b ) + std::max< int64_t >( l_size_k - 1, 0 ) * l_sk_b ) + 64 < ( int64_t( 1 ) << 31 )
      && 2 * int64_t( 64 ) * std::max( l_sk_a, l_sk_b ) * ( ( l_size_k + 63 ) / 64 + 4 ) < ( int64_t( 1 ) << 31 );
  plan.tile_fallback = plan.tile;
  if( l_dma_ok && n_tiles( TILE_BF16_DMA_256x256 ) >= l_cus ) plan.tile = TILE_BF16_DMA_256x256;
  // the fp32 direct-to-LDS kernel: where the planner chose the 128 x 128 fp32
  // tile, under the same conditions (4-byte elements; the loads of the step
  // past the last one are issued too); a K that is not affine up to 1024,
  // whose offset tables the kernel copies into LDS
  int64_t const l_bytes_max = int64_t( 1 ) << 31;
  bool const l_f32_dma_k =
         ( l_k_affine
           && 4 * ( max_of( l_tm_a ) + std::max< int64_t >( l_size_k - 1, 0 ) * l_sk_a ) + 64 < l_bytes_max
           && 4 * ( max_of( l_tn_b ) + std::max< int64_t >( l_size_k - 1, 0 ) * l_sk_b ) + 64 < l_bytes_max
           && 4 * int64_t( 32 ) * std::max( l_sk_a, l_sk_b ) * ( ( l_size_k + 31 ) / 32 + 2 ) < l_bytes_max )
      || ( !l_k_affine && l_size_k <= 1024
           && 4 * ( max_of( l_tm_a ) + max_of( l_tk_a ) ) + 64 < l_bytes_max
           && 4 * ( max_of( l_tn_b ) + max_of( l_tk_b ) ) + 64 < l_bytes_max );
  bool const l_f32_dma_ok =
         l_f32 && !l_cpx
      && ( plan.mode_a == LOAD_VEC_MN || plan.mode_a == LOAD_VEC_K )
      && ( plan.mode_b == LOAD_VEC_MN || plan.mode_b == LOAD_VEC_K )
      && l_f32_dma_k;
  if( l_f32_dma_ok && plan.tile == TILE_F32_128x128 ) plan.tile = TILE_F32_DMA_128x128;
  if( char const * l_env = ( l_f64 || l_cpx ) ? nullptr : std::getenv( "ETIR_TILE" ) ) {
    // diagnostic override of the tile heuristic (must match the dtype)
    int32_t l_t = std::atoi( l_env );
    bool const l_t_f32 = ( l_t == TILE_F32_128x128 || l_t == TILE_F32_64x64
                           || ( l_t == TILE_F32_DMA_128x128 && l_f32_dma_ok ) );
    bool const l_t_dma = ( l_t == TILE_BF16_DMA_256x256 || l_t == TILE_BF16_DMA_256x128 );
    bool const l_t_ok = ( ( ( l_t >= 0 && l_t <= TILE_BF16_DMA_256x128 ) || l_t == TILE_F32_DMA_128x128 )
                          && l_t != TILE_F64_64x64 && l_t_f32 == l_f32 )
                     && ( !l_t_dma || l_dma_ok )
                     && ( l_t != TILE_BF16_DMA_256x128
                          || ( plan.mode_a == LOAD_VEC_MN && plan.mode_b == LOAD_VEC_MN ) );
    if( l_t_ok ) plan.tile = l_t;
  }
  // VEC_MN x VEC_MN runs the explicitly scheduled BK 32 / 4-stage main loop;
  // the other pairings (VEC_K needs 64-wide k rows) the generic BK 64 / 2-stage one
  // (3: the persistent variant of the scheduled loop, for contractions it
  // runs -- all tiles full, plain fp32 stores -- decided at launch)
  plan.dma_variant = ( plan.mode_a == LOAD_VEC_MN && plan.mode_b == LOAD_VEC_MN ) ? 3 : 0;
  if( char const * l_env = std::getenv( "ETIR_DMA_VARIANT" ) ) {
    // diagnostic override, only values whose kernel runs on this plan's
    // 256 x 256 tile grid: 0 forces the generic BK 64 / 2-stage loop, 1 the
    // one-tile scheduled loop and 3 its persistent form (both VEC_MN x
    // VEC_MN only); anything else is ignored (the 256 x 128 kernel has a
    // tile grid of its own and is chosen by ETIR_TILE)
    int32_t const l_v = std::atoi( l_env );
    if( l_v == 0 ) plan.dma_variant = 0;
    if( ( l_v == 1 || l_v == 3 ) && plan.dma_variant == 3 ) plan.dma_variant = l_v;
  }

  // ------------------------------------------------------- matrix-vector
  // One free side of extent 1 pads every MFMA tile to one row in 64: one
  // thread per output element instead, when the long side's operand is
  // unit-stride along it (coalesced loads), K is short enough for a
  // per-thread loop and the outputs fill the chip (256 CUs x 1024 threads).
  // ETIR_TILE=13 forces it for any M == 1 or N == 1 shape.
  {
    bool const l_mv_shape = ( l_f32 || l_bf16 ) && !l_cpx && ( l_kern_m == 1 || l_kern_n == 1 );
    char const * l_env_t = std::getenv( "ETIR_TILE" );
    bool const l_forced = l_mv_shape && l_env_t != nullptr && std::atoi( l_env_t ) == TILE_GEMV;
    bool const l_long_vec = ( l_kern_m == 1 && l_kern_n > 1 ) ? ( plan.mode_b == LOAD_VEC_MN )
                          : ( l_kern_n == 1 && l_kern_m > 1 ) ? ( plan.mode_a == LOAD_VEC_MN ) : false;
    bool const l_mv_ok = l_mv_shape && l_long_vec && l_size_k <= 256
                      && l_size_c * l_kern_m * l_kern_n >= 1024 * l_cus
                      && l_env_t == nullptr && std::getenv( "ETIR_NO_GEMV" ) == nullptr;
    if( l_mv_ok || l_forced ) plan.tile = TILE_GEMV;
  }

  // ------------------------------------------------- one short free side
  // A free side of 2 to 64 pads most of every MFMA tile, and with a short K
  // the tiles are bound by their load round trip and stores: one thread per
  // index of the long side instead, the short side's outputs in registers
  // (einsum_benchmark MERA, M = 11, N = 415800, K = 24: 28 us on 64 x 64
  // tiles).  Where the short side is 17-64, only with K <= 64 (the FMAs per
  // long-operand byte grow with the short side); at least 256 workgroups of
  // 256 threads.  ETIR_TILE=14 forces it for any short side of 2 to 64.
  {
    int64_t const l_sh = std::min( l_kern_m, l_kern_n );
    int64_t const l_lo = std::max( l_kern_m, l_kern_n );
    bool const l_sk_shape = ( l_f32 || l_bf16 ) && !l_cpx && plan.tile != TILE_GEMV && l_sh >= 2 && l_sh <= 64
                         && l_size_c <= 65535;
    char const * l_env_t = std::getenv( "ETIR_TILE" );
    bool const l_forced = l_sk_shape && l_env_t != nullptr && std::atoi( l_env_t ) == TILE_SKINNY;
    // not where the output's unit-stride dim is a C dim: a thread's stores
    // would then be C elements apart (TCCG efbadx,cfx->abcdex: 2.3 against
    // 7.8 TFLOP/s on the tiles, which walk C fastest there)
    int64_t l_os_c = std::numeric_limits< int64_t >::max();
    int64_t l_os_mn = std::numeric_limits< int64_t >::max();
    for( Loop const & l_x : l_c ) if( l_x.size > 1 ) l_os_c = std::min( l_os_c, l_x.s[T_OUT] );
    for( auto const * l_set : { &l_m, &l_n } ) {
      for( Loop const & l_x : *l_set ) if( l_x.size > 1 ) l_os_mn = std::min( l_os_mn, l_x.s[T_OUT] );
    }
    bool const l_sk_ok = l_sk_shape && ( l_sh <= 16 || l_size_k <= 64 ) && l_os_mn < l_os_c
                      && l_size_c * ( ( l_lo + 255 ) / 256 ) >= l_cus && l_env_t == nullptr
                      && std::getenv( "ETIR_NO_SKINNY" ) == nullptr;
    if( l_sk_ok || l_forced ) plan.tile = TILE_SKINNY;
  }

  // ------------------------------------- short K, one free side of 65-256
  // With K <= 64 an MFMA tile lives for one load round trip and its stores
  // (einsum_benchmark MERA root, M = 177147, N = 243, K = 50: 73 us on 128 x
  // 128 tiles, 62 here): the short operand stays in LDS for the whole launch
  // and persistent workgroups stream panels of the long side, each panel's
  // stores issued between the next one's MFMAs.  fp32, no C dims, first
  // touch ZERO, last touch none or RELU, the long operand affine along its
  // side, at least four panels per CU (each workgroup pays about one panel
  // of set-up: M = 16384 k x 243 x 50 at 2 / 4 panels per CU 22.7 / 32.1 us
  // against 21.1 / 40.9 on the tiles).  ETIR_TILE=15 forces it where the
  // shape allows (a long side of at least one panel), ETIR_NO_PANEL turns it
  // off.
  {
    int64_t const l_sh = std::min( l_kern_m, l_kern_n );
    int64_t const l_lo = std::max( l_kern_m, l_kern_n );
    bool const l_res_a = l_kern_m <= l_kern_n;
    std::vector< int64_t > const & l_tl = l_res_a ? l_tn_b : l_tm_a;
    bool l_aff = true;
    int64_t const l_st = l_tl.size() > 1 ? l_tl[1] : 0;
    for( std::size_t l_i = 0; l_i < l_tl.size() && l_aff; l_i++ ) l_aff = ( l_tl[l_i] == int64_t( l_i ) * l_st );
    l_aff = l_aff && l_st >= 0 && l_st <= std::numeric_limits< int32_t >::max();
    int64_t l_mo = 0, l_no = 0;
    for( int64_t l_v : l_tm_out ) l_mo = std::max( l_mo, l_v );
    for( int64_t l_v : l_tn_out ) l_no = std::max( l_no, l_v );
    bool const l_pn_shape = l_f32 && !l_cpx && plan.tile != TILE_GEMV && plan.tile != TILE_SKINNY
                         && l_size_c == 1 && l_sh > 64 && l_sh <= 256 && l_size_k >= 1 && l_size_k <= 64
                         && ktype_first_touch == ETIR_KTYPE_ZERO
                         && ( ktype_last_touch == ETIR_KTYPE_UNDEFINED || ktype_last_touch == ETIR_KTYPE_RELU )
                         && !plan.needs_aux && l_aff && 4 * ( l_mo + l_no + 1 ) <= int64_t( 0xffffff00u );
    int64_t const l_pl = ( l_sh > 128 ) ? 64 : 128;
    char const * l_env_t = std::getenv( "ETIR_TILE" );
    bool const l_forced = l_pn_shape && l_lo >= l_pl && l_env_t != nullptr && std::atoi( l_env_t ) == TILE_PANEL;
    bool const l_pn_ok = l_pn_shape && ( l_lo + l_pl - 1 ) / l_pl >= 4 * l_cus && l_env_t == nullptr
                      && std::getenv( "ETIR_NO_PANEL" ) == nullptr;
    if( l_pn_ok || l_forced ) plan.tile = TILE_PANEL;
  }

  // ------------------------------------------- long K on few large tiles
  // The 64 x 64 tile fills the chip where fewer than 256 of the 128 x 128
  // tiles exist, but runs at about half the fp32 direct-to-LDS kernel's rate;
  // with K >= 2048 the larger tile split over K (below) is faster (1024 x 1024
  // x 8192: 148 us against 198; 1215 x 924 x 4620: 139 against 188).  Undone
  // after the split block if K does not split.
  int32_t const l_tile_unsplit = plan.tile;
  bool const l_big_k_split = allow_split && l_f32_dma_ok && plan.tile == TILE_F32_64x64 && l_size_k >= 2048
                          && n_tiles( TILE_F32_128x128 ) < l_cus && std::getenv( "ETIR_TILE" ) == nullptr;
  if( l_big_k_split ) plan.tile = TILE_F32_DMA_128x128;

  int64_t l_bm, l_bn;
  tile_shape( plan.tile, l_bm, l_bn );

  // --------------------------------------------- K split inside a workgroup
  // Few output tiles, both operands K-contiguous fp32, K up to 4096: 32 x 32
  // tiles (4x the workgroups of 64 x 64) with K divided over the 16 waves of
  // each workgroup, whose partial tiles are added in LDS -- one launch, no
  // workspace (the alternative below, split K, sends S partial outputs
  // through memory to a second kernel).  At most 512 of them, one round of
  // two workgroups per CU (bench_mlp's 576-tile nodes: 95 us/eval with them,
  // 90 on split K)
  {
    int64_t const l_t32 = n_tiles( TILE_F32_KWAVE_32x32 );
    bool const l_kw_ok = l_f32 && plan.tile != TILE_GEMV && plan.tile != TILE_SKINNY && plan.tile != TILE_PANEL && plan.mode_a == LOAD_VEC_K && plan.mode_b == LOAD_VEC_K && l_k_affine
                      && l_sk_a == 1 && l_sk_b == 1 && l_size_k % 16 == 0 && l_size_k >= 256
                      && l_size_k <= 4096 && n_tiles( plan.tile ) < l_cus && l_t32 >= l_cus / 2
                      && l_t32 <= 2 * l_cus
                      && std::getenv( "ETIR_NO_KWAVE" ) == nullptr;
    if( l_kw_ok ) {
      // 8 waves up to K = 512, 16 above (config 1, K = 512: 7.58-7.65 us with
      // 8 waves against 7.85-7.87 with 16 and 8.8 with 4; K = 256 and 1024:
      // 8 and 16 equal within 1 %)
      int32_t const l_w = ( l_size_k <= 512 ) ? 8 : 16;
      plan.tile = TILE_F32_KWAVE_32x32;
      plan.tile_fallback = TILE_F32_64x64;
      plan.kwave_waves = l_w;
      plan.kwave_kw = (int32_t) ( ( ( l_size_k + l_w - 1 ) / l_w + 15 ) / 16 * 16 );
      tile_shape( plan.tile, l_bm, l_bn );
    }
  }

  // ------------------------------------------------------------- split K
  // Few output tiles and a long K leave most CUs idle (e.g. an einsum-tree
  // node with M = 64, N = 1024, K = 32768).  Then the outermost K loops (one
  // of them factored if needed) become C loops of a partial contraction that
  // writes one workspace slice per split, and split_reduce sums the slices.
  if( allow_split && !l_f64 && !l_cpx && l_size_k >= 512 && plan.tile != TILE_F32_KWAVE_32x32
      && plan.tile != TILE_GEMV && plan.tile != TILE_SKINNY && plan.tile != TILE_PANEL ) {
    int64_t const l_tiles = n_tiles( plan.tile );
    if( l_tiles > 0 && l_tiles < l_cus ) {
      // at least 128 k per split; aim for two workgroups per CU
      int64_t const l_smax   = l_size_k / 128;
      int64_t const l_target = std::min( ( 2 * l_cus + l_tiles - 1 ) / l_tiles, l_smax );
      std::vector< Loop > l_kk = l_k;          // K loops, outer -> inner
      std::vector< Loop > l_sp;                // split parts, outer -> inner
      int64_t l_sf = 1;
      std::size_t l_i = 0;
      while( l_sf < l_target && l_i < l_kk.size() ) {
        Loop & l_lp = l_kk[l_i];
        int64_t const l_need = ( l_target + l_sf - 1 ) / l_sf;
        // factor of this loop: the smallest divisor that reaches the target,
        // else the largest one that stays within l_smax
        // (first pass: where this is the innermost K loop and unit-stride in
        // an operand, only factors that leave its inner part a multiple of 4,
        // so that K rows stay 16-byte loadable: 4620 = 4 x 1155 on the fp32
        // direct-to-LDS kernel measured 457 us, 5 x 924 the vector loads)
        int64_t l_f = 0;
        bool const l_keep4 = l_i + 1 == l_kk.size() && l_lp.size % 4 == 0
                          && ( l_lp.s[T_L] == 1 || l_lp.s[T_R] == 1 );
        for( int l_pass = l_keep4 ? 0 : 1; l_pass < 2 && l_f == 0; l_pass++ ) {
          for( int64_t l_d = 2; l_d <= l_lp.size; l_d++ ) {
            if( l_lp.size % l_d != 0 || l_sf * l_d > l_smax ) continue;
            if( l_pass == 0 && ( l_lp.size / l_d ) % 4 != 0 ) continue;
            l_f = l_d;
            if( l_d >= l_need ) break;
          }
        }
        if( l_f == 0 ) break;
        if( l_f == l_lp.size ) {
          l_sp.push_back( l_lp );
          l_sf *= l_lp.size;
          l_lp.size = 1;
          l_i++;
        }
        else {
          // k = ko * (size / f) + ki: the outer part steps over size / f
          Loop l_outer = l_lp;
          int64_t const l_inner = l_lp.size / l_f;
          l_outer.size = l_f;
          for( int l_t = 0; l_t < 4; l_t++ ) l_outer.s[l_t] *= l_inner;
          l_lp.size = l_inner;
          l_sp.push_back( l_outer );
          l_sf *= l_f;
          break;
        }
      }
      // extent of the output (elements) over its C, M and N loops; the
      // workspace slices lie l_span apart, the extent rounded up to 64
      // elements (16-byte aligned slices)
      int64_t l_ext = 1;
      for( auto const * l_set : { &l_c, &l_m, &l_n } ) {
        for( Loop const & l_x : *l_set ) l_ext += ( l_x.size - 1 ) * l_x.s[T_OUT];
      }
      int64_t const l_span = ( l_ext + 63 ) / 64 * 64;
      // dense output: its loops, by output stride, each stride the product
      // of the sizes below it (then the offsets are exactly 0 .. l_ext - 1)
      int64_t l_dense = 0;
      {
        std::vector< std::pair< int64_t, int64_t > > l_ds;
        for( auto const * l_set : { &l_c, &l_m, &l_n } ) {
          for( Loop const & l_x : *l_set ) if( l_x.size > 1 ) l_ds.push_back( { l_x.s[T_OUT], l_x.size } );
        }
        std::sort( l_ds.begin(), l_ds.end() );
        int64_t l_pack = 1;
        bool l_ok = true;
        for( auto const & l_d : l_ds ) {
          l_ok = l_ok && ( l_d.first == l_pack );
          l_pack *= l_d.second;
        }
        if( l_ok && l_pack == l_ext ) l_dense = l_ext;
      }
      // with an aux tensor: every loop either matches the output's stride in
      // the aux tensor or is broadcast (aux stride 0), the broadcast loops
      // outermost in the output; then the aux offset is o % (the extent of
      // the others)
      int64_t l_dense_aux = 0;
      if( l_dense > 0 && plan.needs_aux ) {
        int64_t l_inner = 1;
        int64_t l_bmin = std::numeric_limits< int64_t >::max();
        int64_t l_kmax = 0;
        bool l_ok = true;
        for( auto const * l_set : { &l_c, &l_m, &l_n } ) {
          for( Loop const & l_x : *l_set ) {
            if( l_x.size <= 1 ) continue;
            if( l_x.s[T_AUX] == 0 ) l_bmin = std::min( l_bmin, l_x.s[T_OUT] );
            else {
              l_ok = l_ok && ( l_x.s[T_AUX] == l_x.s[T_OUT] );
              l_inner *= l_x.size;
              l_kmax = std::max( l_kmax, l_x.s[T_OUT] );
            }
          }
        }
        if( l_ok && ( l_bmin == std::numeric_limits< int64_t >::max() || l_bmin == l_inner ) && l_kmax < l_inner ) {
          l_dense_aux = l_inner;
        }
      }
      int64_t const l_ws_bytes = 4 * l_sf * l_span;
      if( l_sf >= 2 && l_size_k / l_sf >= 128 && l_ws_bytes <= ( int64_t( 1 ) << 29 ) ) {
        // loop arrays of the partial contraction
        std::vector< int32_t > l_pt;
        std::vector< int64_t > l_psz, l_pl, l_pr, l_pa, l_po;
        auto add = [&]( int32_t t, int64_t sz, int64_t sl, int64_t sr, int64_t sa, int64_t so ) {
          l_pt.push_back( t ); l_psz.push_back( sz ); l_pl.push_back( sl ); l_pr.push_back( sr );
          l_pa.push_back( sa ); l_po.push_back( so );
        };
        int64_t l_inner_sp = 1;
        for( std::size_t l_j = l_sp.size(); l_j-- > 0; ) {
          Loop const & l_x = l_sp[l_j];
          add( ETIR_DIM_C, l_x.size, l_x.s[T_L], l_x.s[T_R], 0, l_span * l_inner_sp );
          l_inner_sp *= l_x.size;
        }
        for( auto const * l_set : { &l_c, &l_m, &l_n } ) {
          for( Loop const & l_x : *l_set ) add( l_x.type, l_x.size, l_x.s[T_L], l_x.s[T_R], l_x.s[T_AUX], l_x.s[T_OUT] );
        }
        for( Loop const & l_x : l_kk ) {
          if( l_x.size > 1 ) add( ETIR_DIM_K, l_x.size, l_x.s[T_L], l_x.s[T_R], 0, 0 );
        }
        auto l_part = std::make_shared< ContractionPlan >();
        int l_err = plan_contraction_impl( (int64_t) l_pt.size(), l_pt.data(), l_psz.data(), l_pl.data(),
                                           l_pr.data(), l_pa.data(), l_po.data(), dtype_left, dtype_right,
                                           ETIR_FP32, ETIR_FP32, ETIR_KTYPE_ZERO, ETIR_KTYPE_MADD,
                                           ETIR_KTYPE_UNDEFINED, false, *l_part, place );
        if( l_err != ETIR_SUCCESS ) {
          release_contraction( *l_part );
          return l_err;
        }
        if( place != nullptr ) {
          l_err = place_take( *place, (std::size_t) l_ws_bytes, &plan.d_ws, "split-K workspace" );
          if( l_err != ETIR_SUCCESS ) {
            release_contraction( *l_part );
            return l_err;
          }
        }
        else {
          hipError_t l_he = hipMalloc( &plan.d_ws, (std::size_t) l_ws_bytes );
          if( l_he != hipSuccess ) {
            plan.d_ws = nullptr;
            release_contraction( *l_part );
            return fail( ETIR_UNDEFINED_ERROR, std::string( "contraction: workspace allocation failed: " )
                                               + hipGetErrorString( l_he ) );
          }
        }
        plan.split    = (int32_t) l_sf;
        plan.out_span = l_span;
        plan.out_dense     = ( !plan.needs_aux || l_dense_aux > 0 ) ? l_dense : 0;
        plan.out_dense_aux = plan.needs_aux ? l_dense_aux : 0;
        plan.partial  = l_part;
        plan.C = l_size_c;
        plan.M = l_part->M;
        plan.N = l_part->N;
        plan.K = l_size_k;
        plan.mode_a = l_part->mode_a;
        plan.mode_b = l_part->mode_b;
        plan.tile = l_part->tile;
        plan.flops = 2 * l_size_c * l_size_m * l_size_n * l_size_k;
        int64_t const l_esz_o = ( dtype_out == ETIR_BF16 ) ? 2 : 4;
        plan.bytes = l_esz * l_size_c * ( l_size_m + l_size_n ) * l_size_k
                   + l_esz_o * l_size_c * l_size_m * l_size_n;
        plan.desc = "split-K S=" + std::to_string( l_sf ) + " K'=" + std::to_string( l_size_k / l_sf )
                  + " | " + l_part->desc + " | reduce" + ( plan.out_dense > 0 ? " flat" : "" );
        return ETIR_SUCCESS;
      }
    }
  }
  if( l_big_k_split && plan.tile == TILE_F32_DMA_128x128 ) {
    // K did not split (and K over waves did not take the node): back to the
    // tile that fills the chip by itself
    plan.tile = l_tile_unsplit;
    tile_shape( plan.tile, l_bm, l_bn );
  }

  plan.C = l_size_c;
  plan.M = l_kern_m;
  plan.N = l_kern_n;
  plan.K = l_size_k;
  // complex: four real products per complex multiply-add
  plan.flops = ( l_cpx ? 8 : 2 ) * l_size_c * l_size_m * l_size_n * l_size_k;
  int64_t const l_esz_out = ( dtype_out == ETIR_BF16 ) ? 2 : ( dtype_out == ETIR_FP64 ? 8 : 4 );
  bool const l_read_out = ktype_first_touch == ETIR_KTYPE_ADD || ktype_first_touch == ETIR_KTYPE_UNDEFINED;
  plan.bytes = ( l_cpx ? 2 : 1 )
             * (   l_esz * l_size_c * ( l_size_m + l_size_n ) * l_size_k
                 + l_esz_out * l_size_c * l_size_m * l_size_n * ( 1 + ( l_read_out ? 1 : 0 )
                                                                    + ( plan.needs_aux ? 1 : 0 ) ) );

  std::ostringstream l_d;
  l_d << "contract " << tile_str( plan.tile )
      << " C=" << l_size_c << dims_str( l_c )
      << " M=" << plan.M << dims_str( l_km )
      << " N=" << plan.N << dims_str( l_kn )
      << " K=" << plan.K << dims_str( l_k )
      << " A=" << ( l_swap ? "right" : "left" ) << ":" << mode_str( plan.mode_a )
      << " B=" << ( l_swap ? "left" : "right" ) << ":" << mode_str( plan.mode_b )
      << " k_affine=" << ( l_k_affine ? 1 : 0 );
  plan.desc = l_d.str();

  // ------------------------------------------------------ device tables
  // layout: int64 C tables first (8-byte aligned), then int32 tables
  std::vector< int64_t > l_c64;
  l_c64.insert( l_c64.end(), l_tc_a.begin(),   l_tc_a.end() );
  l_c64.insert( l_c64.end(), l_tc_b.begin(),   l_tc_b.end() );
  l_c64.insert( l_c64.end(), l_tc_aux.begin(), l_tc_aux.end() );
  l_c64.insert( l_c64.end(), l_tc_out.begin(), l_tc_out.end() );
  std::vector< int32_t > l_t32;
  auto app32 = [&]( std::vector< int64_t > const & t ) {
    for( int64_t l_v : t ) l_t32.push_back( (int32_t) l_v );
  };
  std::size_t const l_o_tm_a = l_t32.size(); app32( l_tm_a );
  std::size_t const l_o_tm_x = l_t32.size(); app32( l_tm_aux );
  std::size_t const l_o_tm_o = l_t32.size(); app32( l_tm_out );
  std::size_t const l_o_tn_b = l_t32.size(); app32( l_tn_b );
  std::size_t const l_o_tn_x = l_t32.size(); app32( l_tn_aux );
  std::size_t const l_o_tn_o = l_t32.size(); app32( l_tn_out );
  std::size_t const l_o_tk_a = l_t32.size(); app32( l_tk_a );
  std::size_t const l_o_tk_b = l_t32.size(); app32( l_tk_b );

  std::size_t const l_bytes64 = l_c64.size() * sizeof( int64_t );
  std::size_t const l_bytes32 = l_t32.size() * sizeof( int32_t );
  std::size_t const l_total = l_bytes64 + l_bytes32 + 256;
  char * l_base = nullptr;
  if( place != nullptr ) {
    // caller's region: the tables are generated there by a kernel from the
    // same loops (and slots) the host enumerated them from above
    int l_err = place_take( *place, l_total, &plan.d_tables, "offset tables" );
    if( l_err != ETIR_SUCCESS ) return l_err;
    l_base = reinterpret_cast< char * >( plan.d_tables );
    int64_t const l_b = int64_t( l_base - place->base );
    int64_t const l_o32 = l_b + int64_t( l_bytes64 );
    auto fill = [&]( std::vector< Loop > const & dims, std::initializer_list< int > slots,
                     std::initializer_list< int64_t > dst, bool is64 ) -> int {
      if( (int) dims.size() > kFillMaxDims ) {
        return fail( ETIR_COMPILATION_FAILED, "contraction: too many fused loops of one type for the "
                                              "allocation-free entry point" );
      }
      TableFill l_f{};
      l_f.count = 1;
      for( Loop const & l_x : dims ) l_f.count *= l_x.size;
      l_f.ndims = (int32_t) dims.size();
      l_f.ntab = (int32_t) slots.size();
      l_f.is64 = is64 ? 1 : 0;
      for( int l_d = 0; l_d < l_f.ndims; l_d++ ) l_f.sizes[l_d] = dims[l_d].size;
      int l_t = 0;
      for( int l_sl : slots ) {
        for( int l_d = 0; l_d < l_f.ndims; l_d++ ) l_f.strides[l_t][l_d] = dims[l_d].s[l_sl];
        l_t++;
      }
      l_t = 0;
      for( int64_t l_o : dst ) l_f.dst[l_t++] = l_o;
      if( l_f.count == 0 ) return ETIR_SUCCESS;
      return launch_fill_tables( l_f, place->base, place->stream );
    };
    int64_t const l_cs = int64_t( sizeof( int64_t ) ) * l_size_c;
    int l_err2 = fill( l_c, { l_sa, l_sb, T_AUX, T_OUT }, { l_b, l_b + l_cs, l_b + 2 * l_cs, l_b + 3 * l_cs }, true );
    if( l_err2 == ETIR_SUCCESS ) {
      l_err2 = fill( l_km, { l_sa, T_AUX, T_OUT }, { l_o32 + 4 * int64_t( l_o_tm_a ), l_o32 + 4 * int64_t( l_o_tm_x ),
                                                    l_o32 + 4 * int64_t( l_o_tm_o ) }, false );
    }
    if( l_err2 == ETIR_SUCCESS ) {
      l_err2 = fill( l_kn, { l_sb, T_AUX, T_OUT }, { l_o32 + 4 * int64_t( l_o_tn_b ), l_o32 + 4 * int64_t( l_o_tn_x ),
                                                    l_o32 + 4 * int64_t( l_o_tn_o ) }, false );
    }
    if( l_err2 == ETIR_SUCCESS ) {
      l_err2 = fill( l_k, { l_sa, l_sb }, { l_o32 + 4 * int64_t( l_o_tk_a ), l_o32 + 4 * int64_t( l_o_tk_b ) }, false );
    }
    if( l_err2 != ETIR_SUCCESS ) return l_err2;
  }
  else {
    ETIR_HIP_CHECK( hipMalloc( &plan.d_tables, l_total ) );
    l_base = reinterpret_cast< char * >( plan.d_tables );
    hipError_t l_e1 = hipMemcpy( l_base, l_c64.data(), l_bytes64, hipMemcpyHostToDevice );
    hipError_t l_e2 = l_bytes32 > 0
                    ? hipMemcpy( l_base + l_bytes64, l_t32.data(), l_bytes32, hipMemcpyHostToDevice )
                    : hipSuccess;
    if( l_e1 != hipSuccess || l_e2 != hipSuccess ) {
      (void) hipFree( plan.d_tables );
      plan.d_tables = nullptr;
      return fail( ETIR_UNDEFINED_ERROR, "contraction: copying offset tables to the device failed" );
    }
  }

  ContractArgs & a = plan.args;
  a = ContractArgs();
  int64_t const * l_p64 = reinterpret_cast< int64_t const * >( l_base );
  a.tc_a   = l_p64;
  a.tc_b   = l_p64 + l_size_c;
  a.tc_aux = l_p64 + 2 * l_size_c;
  a.tc_out = l_p64 + 3 * l_size_c;
  int32_t const * l_p32 = reinterpret_cast< int32_t const * >( l_base + l_bytes64 );
  a.tm_a   = l_p32 + l_o_tm_a;
  a.tm_aux = l_p32 + l_o_tm_x;
  a.tm_out = l_p32 + l_o_tm_o;
  a.tn_b   = l_p32 + l_o_tn_b;
  a.tn_aux = l_p32 + l_o_tn_x;
  a.tn_out = l_p32 + l_o_tn_o;
  a.tk_a   = l_p32 + l_o_tk_a;
  a.tk_b   = l_p32 + l_o_tk_b;
  a.M = (int32_t) l_kern_m;
  a.N = (int32_t) l_kern_n;
  a.K = (int32_t) l_size_k;
  a.C = (int32_t) l_size_c;
  {
    // a C dim innermost in the output: each workgroup (one C index) would
    // write every C-th element, and the workgroups holding the other C
    // indices of the same output lines would run far apart in time; with C
    // fastest in the workgroup order they run side by side (same XCD, same
    // L2) and complete those lines there
    int64_t l_min_c = std::numeric_limits< int64_t >::max();
    int64_t l_min_mn = std::numeric_limits< int64_t >::max();
    for( Loop const & l_x : l_c ) if( l_x.size > 1 ) l_min_c = std::min( l_min_c, l_x.s[T_OUT] );
    for( auto const * l_set : { &l_m, &l_n } ) {
      for( Loop const & l_x : *l_set ) if( l_x.size > 1 ) l_min_mn = std::min( l_min_mn, l_x.s[T_OUT] );
    }
    a.c_inner = ( l_size_c > 1 && l_min_c < l_min_mn ) ? 1 : 0;
    if( a.c_inner ) plan.desc += " c_inner";
  }
  a.tiles_m = (int32_t) ( ( l_kern_m + l_bm - 1 ) / l_bm );
  a.tiles_n = (int32_t) ( ( l_kern_n + l_bn - 1 ) / l_bn );
  a.k_affine = l_k_affine ? 1 : 0;
  a.sk_a = (int32_t) l_sk_a;
  a.sk_b = (int32_t) l_sk_b;
  a.first_touch = ktype_first_touch;
  a.last_touch  = ktype_last_touch;
  a.out_bf16 = ( dtype_out == ETIR_BF16 ) ? 1 : 0;
  // start-time stagger of the persistent direct-to-LDS kernel: 4 phases, 3
  // units (~3 us) apart (measured on config 3; diagnostic override by env)
  a.dma_phases = 4;
  a.dma_stagger = 3;
  if( char const * l_env = std::getenv( "ETIR_DMA_PHASES" ) ) a.dma_phases = std::atoi( l_env );
  if( char const * l_env = std::getenv( "ETIR_DMA_STAGGER" ) ) a.dma_stagger = std::atoi( l_env );
  auto affine_stride = []( std::vector< int64_t > const & t ) -> int32_t {
    int64_t const l_st = t.size() > 1 ? t[1] : 0;
    for( std::size_t l_i = 0; l_i < t.size(); l_i++ ) {
      if( t[l_i] != int64_t( l_i ) * l_st ) return -1;
    }
    return ( l_st >= 0 && l_st <= std::numeric_limits< int32_t >::max() ) ? int32_t( l_st ) : -1;
  };
  a.sm_a   = affine_stride( l_tm_a );
  a.sn_b   = affine_stride( l_tn_b );
  a.sm_out = affine_stride( l_tm_out );
  a.sn_out = affine_stride( l_tn_out );
  a.gemv_v4 = ( plan.tile == TILE_GEMV && l_tm_out.size() == 1 && l_tn_out.size() % 4 == 0 && a.sn_b == 1
                && a.sn_out == 1 && all_multiple( l_tc_b, 4 ) && all_multiple( l_tk_b, 4 )
                && all_multiple( l_tc_out, 4 ) && all_multiple( l_tm_out, 4 ) ) ? 1 : 0;
  if( a.gemv_v4 ) plan.desc += " v4";
  {
    bool const l_short_a = l_kern_m <= l_kern_n;
    std::vector< int64_t > const & l_tl = l_short_a ? l_tn_b : l_tm_a;
    std::vector< int64_t > const & l_tcl = l_short_a ? l_tc_b : l_tc_a;
    int64_t const l_skl = l_short_a ? l_sk_b : l_sk_a;
    a.skinny_kvec = ( plan.tile == TILE_SKINNY && l_k_affine && ( l_size_k <= 1 || l_skl == 1 ) && l_size_k % 4 == 0
                      && all_multiple( l_tl, 4 ) && all_multiple( l_tcl, 4 ) ) ? 1 : 0;
    if( a.skinny_kvec ) plan.desc += " kvec";
    // the output as [long][short] with the short side unit-stride (short
    // offsets s, long offsets i * S): a workgroup's outputs are one block,
    // written in address order through LDS; only where the output is
    // written, not read (no accumulation, no aux)
    std::vector< int64_t > const & l_tlo = l_short_a ? l_tn_out : l_tm_out;
    std::vector< int64_t > const & l_tso = l_short_a ? l_tm_out : l_tn_out;
    a.skinny_blk = 0;
    if( plan.tile == TILE_SKINNY && ktype_first_touch == ETIR_KTYPE_ZERO && !plan.needs_aux
        && ( ktype_last_touch == ETIR_KTYPE_UNDEFINED || ktype_last_touch == ETIR_KTYPE_RELU )
        && affine_stride( l_tso ) == 1 ) {
      int64_t const l_s = int64_t( l_tso.size() );
      bool l_ok = true;
      for( std::size_t l_i = 0; l_ok && l_i < l_tlo.size(); l_i++ ) l_ok = ( l_tlo[l_i] == int64_t( l_i ) * l_s );
      if( l_ok ) {
        a.skinny_blk = 1;
        plan.desc += " blk";
      }
    }
  }
  if( l_cpx ) {
    a.cpx_a   = l_x[0].s[l_sa];
    a.cpx_b   = l_x[0].s[l_sb];
    a.cpx_out = l_x[0].s[T_OUT];
  }
  {
    int64_t l_mo = 0, l_no = 0;
    for( int64_t l_v : l_tm_out ) l_mo = std::max( l_mo, l_v );
    for( int64_t l_v : l_tn_out ) l_no = std::max( l_no, l_v );
    a.out_off32 = ( 4 * ( l_mo + l_no ) + 4 < ( int64_t( 1 ) << 32 ) ) ? 1 : 0;
    // non-temporal output stores only where each store instruction of the
    // fast epilogue (32 consecutive columns per half-wave) writes whole
    // unit-stride runs: the output's columns are consecutive in groups of 32
    std::size_t l_run = 1;
    while( l_run < l_tn_out.size() && l_tn_out[l_run] == l_tn_out[l_run - 1] + 1 ) l_run++;
    a.out_nt = ( l_run >= 32 && ( l_run % 32 == 0 || l_run == l_tn_out.size() ) ) ? 1 : 0;
    if( char const * l_env = std::getenv( "ETIR_OUT_NT" ) ) a.out_nt = std::atoi( l_env ) != 0 ? 1 : 0;
  }
  if( plan.tile == TILE_PANEL ) {
    int64_t l_mo = 0, l_no = 0;
    for( int64_t l_v : l_tm_out ) l_mo = std::max( l_mo, l_v );
    for( int64_t l_v : l_tn_out ) l_no = std::max( l_no, l_v );
    a.out_bytes  = uint32_t( 4 * ( l_mo + l_no + 1 ) );
    a.panel_grid = int32_t( l_cus );
  }
  if(    plan.tile == TILE_BF16_DMA_256x256 && plan.dma_variant == 3 && a.M % 256 == 0 && a.N % 256 == 0
      && a.out_off32 && a.out_nt && !a.out_bf16 && a.first_touch == ETIR_KTYPE_ZERO
      && a.last_touch == ETIR_KTYPE_UNDEFINED ) {
    plan.desc += " persistent";
  }
  return ETIR_SUCCESS;
}

}  // namespace

int plan_contraction( int64_t            num_loops,
                      int32_t const    * dim_types,
                      int64_t const    * sizes,
                      int64_t const    * strides_left,
                      int64_t const    * strides_right,
                      int64_t const    * strides_out_aux,
                      int64_t const    * strides_out,
                      int32_t            dtype_left,
                      int32_t            dtype_right,
                      int32_t            dtype_comp,
                      int32_t            dtype_out,
                      int32_t            ktype_first_touch,
                      int32_t            ktype_main,
                      int32_t            ktype_last_touch,
                      ContractionPlan  & plan,
                      DevicePlacement  * place ) {
  return plan_contraction_impl( num_loops, dim_types, sizes, strides_left, strides_right, strides_out_aux,
                                strides_out, dtype_left, dtype_right, dtype_comp, dtype_out,
                                ktype_first_touch, ktype_main, ktype_last_touch,
                                std::getenv( "ETIR_NO_SPLIT_K" ) == nullptr, plan, place );
}

void release_contraction( ContractionPlan & plan ) {
  if( !plan.placed && plan.d_tables != nullptr ) (void) hipFree( plan.d_tables );
  if( !plan.placed && plan.d_ws != nullptr ) (void) hipFree( plan.d_ws );
  plan.d_tables = nullptr;
  plan.d_ws = nullptr;
  if( plan.partial ) {
    release_contraction( *plan.partial );
    plan.partial.reset();
  }
}

int launch_contraction( ContractionPlan const & plan,
                        void const            * left,
                        void const            * right,
                        void const            * out_aux,
                        void                  * out,
                        hipStream_t             stream ) {
  if( plan.C == 0 || plan.M == 0 || plan.N == 0 ) return ETIR_SUCCESS;
  if( out == nullptr || ( plan.K > 0 && ( left == nullptr || right == nullptr ) ) ) {
    return fail( ETIR_NO_DATA_PTR_PROVIDED, "contraction: null tensor pointer" );
  }
  if( plan.needs_aux && out_aux == nullptr ) {
    return fail( ETIR_NO_DATA_PTR_PROVIDED, "contraction: touch kernel needs the auxiliary tensor" );
  }
  if( plan.split > 1 ) {
    int l_err = launch_contraction( *plan.partial, left, right, nullptr, plan.d_ws, stream );
    if( l_err != ETIR_SUCCESS ) return l_err;
    ContractArgs const & p = plan.partial->args;
    SplitReduceArgs r{};
    r.ws = reinterpret_cast< float const * >( plan.d_ws );
    r.aux = plan.needs_aux ? out_aux : nullptr;
    r.out = out;
    r.tc_out = p.tc_out;              // the first C entries belong to split 0
    r.tc_aux = p.tc_aux;
    r.tm_out = p.tm_out;
    r.tm_aux = p.tm_aux;
    r.tn_out = p.tn_out;
    r.tn_aux = p.tn_aux;
    r.span = plan.out_span;
    r.n_flat = plan.out_dense;
    r.flat_aux = plan.out_dense_aux;
    r.flat_vec = ( r.n_flat > 0 && r.span % 4 == 0
                   && reinterpret_cast< uintptr_t >( out ) % uintptr_t( plan.dtype_out == ETIR_BF16 ? 8 : 16 ) == 0 ) ? 1 : 0;
    r.C = (int32_t) plan.C;
    r.M = p.M;
    r.N = p.N;
    r.S = plan.split;
    r.first_touch = plan.first_touch;
    r.last_touch = plan.last_touch;
    r.out_bf16 = ( plan.dtype_out == ETIR_BF16 ) ? 1 : 0;
    l_err = launch_split_reduce( r, stream );
    if( l_err != ETIR_SUCCESS ) return l_err;
    hipError_t l_he = hipGetLastError();
    if( l_he != hipSuccess ) {
      return fail( ETIR_UNDEFINED_ERROR, std::string( "split reduce launch failed: " ) + hipGetErrorString( l_he ) );
    }
    return ETIR_SUCCESS;
  }
  ContractArgs a = plan.args;
  a.a   = plan.swapped ? right : left;
  a.b   = plan.swapped ? left : right;
  a.aux = plan.needs_aux ? out_aux : nullptr;
  a.out = out;

  // vector paths need aligned base pointers; otherwise fall back to gathers
  int32_t l_ma = plan.mode_a;
  int32_t l_mb = plan.mode_b;
  int64_t const l_esz = ( plan.dtype_in == ETIR_BF16 ) ? 2 : ( plan.dtype_in == ETIR_FP64 ? 8 : 4 );
  auto align_of = [&]( int32_t mode ) -> uintptr_t {
    if( mode == LOAD_VEC_K || mode == LOAD_VEC_MN ) return 16;
    if( mode == LOAD_VEC8_K || mode == LOAD_VEC8_MN ) return 8;
    return uintptr_t( l_esz );
  };
  if( uintptr_t( a.a ) % align_of( l_ma ) != 0 ) l_ma = LOAD_SCALAR;
  if( uintptr_t( a.b ) % align_of( l_mb ) != 0 ) l_mb = LOAD_SCALAR;
  int32_t l_dma_variant = plan.dma_variant;
  int32_t l_tile = plan.tile;
  if(    ( l_tile == TILE_BF16_DMA_256x256 || l_tile == TILE_BF16_DMA_256x128 || l_tile == TILE_F32_KWAVE_32x32
           || l_tile == TILE_F32_DMA_128x128 )
      && ( l_ma != plan.mode_a || l_mb != plan.mode_b ) ) {
    // the DMA and K-over-waves kernels need the 16-byte vector modes: use
    // the register-staged kernel with its own tile grid
    l_tile = plan.tile_fallback;
    int64_t l_bm, l_bn;
    tile_shape( l_tile, l_bm, l_bn );
    a.tiles_m = (int32_t) ( ( plan.M + l_bm - 1 ) / l_bm );
    a.tiles_n = (int32_t) ( ( plan.N + l_bn - 1 ) / l_bn );
  }

  int64_t const l_grid = int64_t( a.tiles_m ) * a.tiles_n * a.C;
  if( l_grid > 0x7fffffffLL ) {
    return fail( ETIR_UNDEFINED_ERROR, "contraction: grid too large" );
  }
  bool const l_kaff = ( a.k_affine != 0 );
  uint32_t const l_g = (uint32_t) l_grid;
  int l_err;
  switch( l_tile ) {
    case TILE_F32_128x128:
    case TILE_F32_64x64:
    case TILE_BF16_256x256:
    case TILE_BF16_256x128:
    case TILE_BF16_128x128:
    case TILE_BF16_64x64:
      l_err = launch_contract_tile( l_tile, l_ma, l_mb, l_kaff, a, l_g, stream );
      break;
    case TILE_F64_64x64:    l_err = launch_contract_f64_64x64( l_ma, l_mb, l_kaff, a, l_g, stream ); break;
    case TILE_CPX_F32_64x64: l_err = launch_contract_cpx( false, l_ma, l_mb, l_kaff, a, l_g, stream ); break;
    case TILE_CPX_F64_64x64: l_err = launch_contract_cpx( true, l_ma, l_mb, l_kaff, a, l_g, stream ); break;
    case TILE_F32_KWAVE_32x32:
      l_err = launch_contract_kwave( plan.kwave_waves, plan.kwave_kw, a, l_g, stream );
      break;
    case TILE_BF16_DMA_256x256:
      l_err = launch_contract_bf16_dma( l_ma, l_mb, l_dma_variant, a, l_g, stream );
      break;
    case TILE_BF16_DMA_256x128:
      l_err = launch_contract_bf16_dma( l_ma, l_mb, 2, a, l_g, stream );
      break;
    case TILE_F32_DMA_128x128:
      l_err = launch_contract_f32_dma( l_ma, l_mb, a, l_g, stream );
      break;
    case TILE_GEMV:
      l_err = launch_contract_gemv( plan.dtype_in == ETIR_BF16, a, stream );
      break;
    case TILE_SKINNY:
      l_err = launch_contract_skinny( plan.dtype_in == ETIR_BF16, a, stream );
      break;
    case TILE_PANEL:
      l_err = launch_contract_panel( a, stream );
      break;
    default: return fail( ETIR_COMPILATION_FAILED, "contraction: unknown tile configuration" );
  }
  if( l_err != ETIR_SUCCESS ) return l_err;
  hipError_t l_he = hipGetLastError();
  if( l_he != hipSuccess ) {
    return fail( ETIR_UNDEFINED_ERROR, std::string( "contraction launch failed: " ) + hipGetErrorString( l_he ) );
  }
  return ETIR_SUCCESS;
}

}  // namespace etir
