#include "BinaryPrimitives.h"
#include "BinaryContraction.h"
#include <algorithm>

void einsum_ir::backend::BinaryPrimitives::init( int64_t i_size_cb_min, int64_t i_size_cb_max,
                                                 int64_t i_size_mb_min, int64_t i_size_mb_max,
                                                 int64_t i_size_nb_min, int64_t i_size_nb_max,
                                                 int64_t i_size_kb_min, int64_t i_size_kb_max ) {
  m_size_cb_min = i_size_cb_min;  m_size_cb_max = i_size_cb_max;
  m_size_mb_min = i_size_mb_min;  m_size_mb_max = i_size_mb_max;
  m_size_nb_min = i_size_nb_min;  m_size_nb_max = i_size_nb_max;
  m_size_kb_min = i_size_kb_min;  m_size_kb_max = i_size_kb_max;
}

einsum_ir::err_t einsum_ir::backend::BinaryPrimitives::init( data_t    i_data_type,
                                                             backend_t i_backend_type ) {
  // TPP targets of the reference (BinaryPrimitives.cpp:28-44); the HIP backend
  // uses the same tensor ordering and targets, so a tree is laid out exactly
  // as on the reference's TPP path (bf16 takes the fp32 targets).
  bool const l_tpp_like = ( i_backend_type == backend_t::TPP || i_backend_type == backend_t::HIP );
  bool const l_blas_like = ( i_backend_type == backend_t::BLAS || i_backend_type == backend_t::TBLIS );
  if( l_tpp_like ) {
    if( i_data_type == data_t::FP32 || i_data_type == data_t::BF16 ) {
      init( 4, 16, 32, 128, 12, 64, 32, 512 );
    }
    else if( i_data_type == data_t::FP64 ) {
      init( 2, 8, 16, 64, 6, 32, 16, 256 );
    }
    else {
      return err_t::INVALID_DTYPE;
    }
  }
  else if( l_blas_like ) {
    if( i_data_type == data_t::FP32 ) {
      init( 4, 16, 32, 512, 32, 512, 32, 512 );
    }
    else if( i_data_type == data_t::FP64 ) {
      init( 2, 8, 16, 256, 16, 256, 16, 256 );
    }
    else {
      return err_t::INVALID_DTYPE;
    }
  }
  else {
    return err_t::INVALID_BACKEND;
  }
  return err_t::SUCCESS;
}

bool einsum_ir::backend::BinaryPrimitives::swap_inputs( int64_t         i_num_dims_left,
                                                        int64_t         i_num_dims_right,
                                                        int64_t         i_num_dims_out,
                                                        int64_t const * i_dim_ids_left,
                                                        int64_t const * i_dim_ids_right,
                                                        int64_t const * i_dim_ids_out ) {
  std::vector< dim_t > l_types_left, l_types_right, l_types_out;
  BinaryContraction::dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
                                i_dim_ids_left, i_dim_ids_right, i_dim_ids_out,
                                &l_types_left, &l_types_right, &l_types_out );
  if( l_types_out.empty() ) return false;
  // fastest output dim is N: swap
  if( l_types_out.back() == N ) return true;
  // fastest output dim is C: the first M or N dim further out decides
  if( l_types_out.back() == C ) {
    for( int64_t l_di = (int64_t) l_types_out.size() - 1; l_di >= 0; l_di-- ) {
      if( l_types_out[l_di] == M ) return false;
      if( l_types_out[l_di] == N ) return true;
    }
  }
  return false;
}

einsum_ir::err_t einsum_ir::backend::BinaryPrimitives::reorder_generic( CBlock                               i_cblock,
                                                                        int64_t                              i_size_cb_min,
                                                                        int64_t                              i_size_cb_max,
                                                                        int64_t                              i_size_mb_min,
                                                                        int64_t                              i_size_mb_max,
                                                                        int64_t                              i_size_nb_min,
                                                                        int64_t                              i_size_nb_max,
                                                                        int64_t                              i_size_kb_min,
                                                                        int64_t                              i_size_kb_max,
                                                                        int64_t                              i_num_dims_left,
                                                                        int64_t                              i_num_dims_right,
                                                                        int64_t                              i_num_dims_out,
                                                                        std::map< int64_t, int64_t > const * i_dim_sizes,
                                                                        int64_t                            * io_dim_ids_left,
                                                                        int64_t                            * io_dim_ids_right,
                                                                        int64_t                            * io_dim_ids_out ) {
  std::vector< dim_t > l_t_left, l_t_right, l_t_out;
  BinaryContraction::dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
                                io_dim_ids_left, io_dim_ids_right, io_dim_ids_out,
                                &l_t_left, &l_t_right, &l_t_out );
  auto size_of = [i_dim_sizes]( int64_t i_id ) { return i_dim_sizes->at( i_id ); };

  std::vector< int64_t > l_cb, l_mb, l_nb, l_kb;          // blocked groups
  std::vector< int64_t > l_bc, l_bm, l_bn, l_bk, l_bi, l_bj;   // the rest

  int64_t l_di = i_num_dims_out - 1;

  // takes trailing output dims of type i_type into o_block while the block
  // is below its minimum or stays within its maximum
  auto take_block = [&]( dim_t i_type, int64_t i_min, int64_t i_max, bool i_unlimited,
                         std::vector< int64_t > & o_block ) {
    int64_t l_block = 1;
    while( l_di >= 0 && l_t_out[l_di] == i_type ) {
      int64_t l_size = size_of( io_dim_ids_out[l_di] );
      if( !i_unlimited && !( l_block < i_min || l_block * l_size <= i_max ) ) break;
      l_block *= l_size;
      o_block.push_back( io_dim_ids_out[l_di] );
      l_di--;
    }
  };

  if( i_cblock == CBlock::INNER ) take_block( C, i_size_cb_min, i_size_cb_max, false, l_cb );
  if( i_cblock == CBlock::OUTER ) take_block( C, 0, 0, true, l_cb );
  take_block( M, i_size_mb_min, i_size_mb_max, false, l_mb );

  // skip C and M dims up to the first N dim
  while( l_di >= 0 && l_t_out[l_di] != N ) {
    if(      l_t_out[l_di] == C ) l_bc.push_back( io_dim_ids_out[l_di] );
    else if( l_t_out[l_di] == M ) l_bm.push_back( io_dim_ids_out[l_di] );
    else return err_t::DIMENSION_ORDERING_FAILED;
    l_di--;
  }
  take_block( N, i_size_nb_min, i_size_nb_max, false, l_nb );
  while( l_di >= 0 ) {
    if(      l_t_out[l_di] == C ) l_bc.push_back( io_dim_ids_out[l_di] );
    else if( l_t_out[l_di] == M ) l_bm.push_back( io_dim_ids_out[l_di] );
    else if( l_t_out[l_di] == N ) l_bn.push_back( io_dim_ids_out[l_di] );
    else return err_t::DIMENSION_ORDERING_FAILED;
    l_di--;
  }

  // K dims, largest first; the leading ones form the K block
  std::vector< int64_t > l_k;
  for( int64_t l_i = 0; l_i < i_num_dims_left; l_i++ ) {
    if( l_t_left[l_i] == K ) l_k.push_back( io_dim_ids_left[l_i] );
  }
  // size order with ties in reverse input order: the order the reference's
  // std::sort with a non-strict comparator produces on these short lists
  // (insertion sort moves an equal later element in front of earlier ones)
  std::reverse( l_k.begin(), l_k.end() );
  std::stable_sort( l_k.begin(), l_k.end(),
                    [&]( int64_t i_a, int64_t i_b ) { return size_of( i_a ) > size_of( i_b ); } );
  int64_t l_block = 1;
  std::size_t l_nkb = 0;
  for( ; l_nkb < l_k.size(); l_nkb++ ) {
    int64_t l_size = size_of( l_k[l_nkb] );
    if( !( l_block < i_size_kb_min || l_block * l_size <= i_size_kb_max ) ) break;
    l_block *= l_size;
  }
  l_kb.assign( l_k.begin(), l_k.begin() + l_nkb );
  l_bk.assign( l_k.begin() + l_nkb, l_k.end() );

  // I and J dims, smallest first
  for( int64_t l_i = 0; l_i < i_num_dims_left; l_i++ ) {
    if( l_t_left[l_i] == I ) l_bi.push_back( io_dim_ids_left[l_i] );
  }
  for( int64_t l_i = 0; l_i < i_num_dims_right; l_i++ ) {
    if( l_t_right[l_i] == J ) l_bj.push_back( io_dim_ids_right[l_i] );
  }
  auto by_size_asc = [&]( int64_t i_a, int64_t i_b ) { return size_of( i_a ) < size_of( i_b ); };
  std::reverse( l_bi.begin(), l_bi.end() );
  std::reverse( l_bj.begin(), l_bj.end() );
  std::stable_sort( l_bi.begin(), l_bi.end(), by_size_asc );
  std::stable_sort( l_bj.begin(), l_bj.end(), by_size_asc );

  // fill both inputs from their fastest position outwards
  int64_t l_pl = i_num_dims_left  - 1;
  int64_t l_pr = i_num_dims_right - 1;
  auto to_left  = [&]( std::vector< int64_t > const & i_ids ) { for( int64_t l_id : i_ids ) io_dim_ids_left[l_pl--]  = l_id; };
  auto to_right = [&]( std::vector< int64_t > const & i_ids ) { for( int64_t l_id : i_ids ) io_dim_ids_right[l_pr--] = l_id; };
  auto to_both  = [&]( std::vector< int64_t > const & i_ids ) { to_left( i_ids ); to_right( i_ids ); };

  if( i_cblock == CBlock::INNER ) to_both( l_cb );
  to_left( l_mb );
  to_both( l_kb );
  to_right( l_nb );
  if( i_cblock == CBlock::OUTER ) to_both( l_cb );
  to_left( l_bi );
  to_right( l_bj );
  to_both( l_bk );
  to_left( l_bm );
  to_right( l_bn );
  to_both( l_bc );

  if( l_pl != -1 || l_pr != -1 ) return err_t::DIMENSION_ORDERING_FAILED;
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::BinaryPrimitives::reorder( tenord_t                             i_primitive_ordering,
                                                                int64_t                              i_num_dims_left,
                                                                int64_t                              i_num_dims_right,
                                                                int64_t                              i_num_dims_out,
                                                                std::map< int64_t, int64_t > const * i_dim_sizes,
                                                                int64_t                            * io_dim_ids_left,
                                                                int64_t                            * io_dim_ids_right,
                                                                int64_t                            * io_dim_ids_out ) const {
  CBlock l_cb;
  if(      i_primitive_ordering == tenord_t::LEFT_NATIVE_RIGHT_NATIVE_OUT_NATIVE ) return err_t::SUCCESS;
  else if( i_primitive_ordering == tenord_t::LEFT_BC_BM_BK_BI_KB_MB_RIGHT_BC_BN_BK_BJ_NB_KB_OUT_NATIVE ) l_cb = CBlock::NONE;
  else if( i_primitive_ordering == tenord_t::LEFT_BC_BM_BK_BI_KB_MB_CB_RIGHT_BC_BN_BK_BJ_NB_KB_CB_OUT_NATIVE ) l_cb = CBlock::INNER;
  else if( i_primitive_ordering == tenord_t::LEFT_BC_BM_BK_BI_CB_KB_MB_RIGHT_BC_BN_BK_BJ_CB_NB_KB_OUT_NATIVE ) l_cb = CBlock::OUTER;
  else return err_t::DIMENSION_ORDERING_FAILED;

  return reorder_generic( l_cb,
                          m_size_cb_min, m_size_cb_max, m_size_mb_min, m_size_mb_max,
                          m_size_nb_min, m_size_nb_max, m_size_kb_min, m_size_kb_max,
                          i_num_dims_left, i_num_dims_right, i_num_dims_out, i_dim_sizes,
                          io_dim_ids_left, io_dim_ids_right, io_dim_ids_out );
}

einsum_ir::err_t einsum_ir::backend::BinaryPrimitives::reorder( backend_t                            i_backend_type,
                                                                int64_t                              i_num_dims_left,
                                                                int64_t                              i_num_dims_right,
                                                                int64_t                              i_num_dims_out,
                                                                std::map< int64_t, int64_t > const * i_dim_sizes,
                                                                int64_t                            * io_dim_ids_left,
                                                                int64_t                            * io_dim_ids_right,
                                                                int64_t                            * io_dim_ids_out ) const {
  std::vector< dim_t > l_t_left, l_t_right, l_t_out;
  BinaryContraction::dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
                                io_dim_ids_left, io_dim_ids_right, io_dim_ids_out,
                                &l_t_left, &l_t_right, &l_t_out );
  if( i_backend_type == backend_t::HIP ) {
    // both children laid out for the GPU kernel (fp32 vector width)
    return reorder_gpu( false, false, 4, 4, 0, i_num_dims_left, i_num_dims_right, i_num_dims_out,
                        i_dim_sizes, io_dim_ids_left, io_dim_ids_right, io_dim_ids_out );
  }
  tenord_t l_ord = tenord_t::LEFT_NATIVE_RIGHT_NATIVE_OUT_NATIVE;
  if( i_backend_type == backend_t::TPP || i_backend_type == backend_t::TBLIS ) {
    l_ord = tenord_t::LEFT_BC_BM_BK_BI_KB_MB_CB_RIGHT_BC_BN_BK_BJ_NB_KB_CB_OUT_NATIVE;
  }
  else if( i_backend_type == backend_t::BLAS ) {
    l_ord = ( !l_t_out.empty() && l_t_out.back() == C )
          ? tenord_t::LEFT_BC_BM_BK_BI_CB_KB_MB_RIGHT_BC_BN_BK_BJ_CB_NB_KB_OUT_NATIVE
          : tenord_t::LEFT_BC_BM_BK_BI_KB_MB_CB_RIGHT_BC_BN_BK_BJ_NB_KB_CB_OUT_NATIVE;
  }
  return reorder( l_ord, i_num_dims_left, i_num_dims_right, i_num_dims_out, i_dim_sizes,
                  io_dim_ids_left, io_dim_ids_right, io_dim_ids_out );
}

einsum_ir::err_t einsum_ir::backend::BinaryPrimitives::reorder_gpu( bool                                 i_fixed_left,
                                                                    bool                                 i_fixed_right,
                                                                    int64_t                              i_vec,
                                                                    int64_t                              i_bytes_per_element,
                                                                    int64_t                              i_min_bytes_permute,
                                                                    int64_t                              i_num_dims_left,
                                                                    int64_t                              i_num_dims_right,
                                                                    int64_t                              i_num_dims_out,
                                                                    std::map< int64_t, int64_t > const * i_dim_sizes,
                                                                    int64_t                            * io_dim_ids_left,
                                                                    int64_t                            * io_dim_ids_right,
                                                                    int64_t                            * io_dim_ids_out ) {
  std::vector< dim_t > l_t[2], l_t_out;
  BinaryContraction::dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
                                io_dim_ids_left, io_dim_ids_right, io_dim_ids_out,
                                &l_t[0], &l_t[1], &l_t_out );
  int64_t * l_ids[2] = { io_dim_ids_left, io_dim_ids_right };
  int64_t const l_nd[2] = { i_num_dims_left, i_num_dims_right };
  bool const l_fixed[2] = { i_fixed_left, i_fixed_right };
  dim_t const l_own[2] = { dim_t::M, dim_t::N };
  auto size_of = [&]( int64_t i_id ) -> int64_t {
    auto l_it = i_dim_sizes->find( i_id );
    return l_it != i_dim_sizes->end() ? l_it->second : 1;
  };

  // the kernel's column side holds the output's unit-stride dim: the left
  // operand if that dim is an M dim (the planner then swaps the roles)
  int64_t const l_o_last = i_num_dims_out > 0 ? io_dim_ids_out[i_num_dims_out - 1] : -1;
  int const l_col_side = ( i_num_dims_out > 0 && l_t_out.back() == dim_t::M ) ? 0 : 1;

  // extents of each child's own M/N dims and of the K dims, and its bytes
  int64_t l_ext_mn[2] = { 1, 1 };
  int64_t l_ext_k = 1;
  int64_t l_bytes[2] = { i_bytes_per_element, i_bytes_per_element };
  for( int l_s = 0; l_s < 2; l_s++ ) {
    for( int64_t l_d = 0; l_d < l_nd[l_s]; l_d++ ) {
      int64_t const l_sz = size_of( l_ids[l_s][l_d] );
      l_bytes[l_s] *= l_sz;
      if( l_t[l_s][l_d] == l_own[l_s] ) l_ext_mn[l_s] *= l_sz;
      if( l_s == 0 && l_t[l_s][l_d] == dim_t::K ) l_ext_k *= l_sz;
    }
  }

  // the output's unit-stride run on the column side (its trailing dims of
  // the column side's type) and its innermost row-side dim: when the run is
  // shorter than a 32-lane store row, consecutive tile rows have to be
  // neighbours in memory for the stores to fill whole lines -- worth a new
  // layout of the row-side child only when the output outweighs that child
  // (TCCG dega,gfbc->abcdef, 1 MB child, 442 MB output: 38 against 22-33
  // TFLOP/s; bda,dc->abc, 226 MB child, 14 MB output: kept, 17 -> 34)
  dim_t const l_col_type = l_own[l_col_side];
  int64_t l_col_run = 1;
  for( int64_t l_o = i_num_dims_out - 1; l_o >= 0 && l_t_out[l_o] == l_col_type; l_o-- ) {
    l_col_run *= size_of( io_dim_ids_out[l_o] );
  }
  int64_t l_o_row_last = -1;
  for( int64_t l_o = i_num_dims_out - 1; l_o >= 0; l_o-- ) {
    if( l_t_out[l_o] == l_own[1 - l_col_side] ) {
      l_o_row_last = io_dim_ids_out[l_o];
      break;
    }
  }

  int64_t l_bytes_out = i_bytes_per_element;
  for( int64_t l_o = 0; l_o < i_num_dims_out; l_o++ ) l_bytes_out *= size_of( io_dim_ids_out[l_o] );
  // per child: 0 = lay out again, 1 = keep (read along M/N), 2 = keep (read
  // along K), 3 = keep (gathered: little data)
  int l_keep[2] = { 0, 0 };
  for( int l_s = 0; l_s < 2; l_s++ ) {
    if( !l_fixed[l_s] || l_nd[l_s] == 0 ) continue;
    int64_t const l_in = l_ids[l_s][l_nd[l_s] - 1];
    dim_t const l_ty = l_t[l_s][l_nd[l_s] - 1];
    // a K dim innermost is read in vectors along the run of the child's
    // trailing K dims, which the planner fuses when the other child holds
    // them in the same order back to back (a child laid out here takes this
    // one's K order); bench_mlp's input, K = 8 x 98: 16-byte loads as it is
    int64_t l_run = size_of( l_in );
    if( l_ty == dim_t::K ) {
      int const l_o = 1 - l_s;
      int64_t l_pos = -1;
      for( int64_t l_d = 0; l_d < l_nd[l_o]; l_d++ ) if( l_ids[l_o][l_d] == l_in ) l_pos = l_d;
      for( int64_t l_q = 1; l_q < l_nd[l_s]; l_q++ ) {
        int64_t const l_d = l_nd[l_s] - 1 - l_q;
        if( l_t[l_s][l_d] != dim_t::K ) break;
        if( l_fixed[l_o] && ( l_pos - l_q < 0 || l_ids[l_o][l_pos - l_q] != l_ids[l_s][l_d] ) ) break;
        l_run *= size_of( l_ids[l_s][l_d] );
      }
    }
    bool const l_vec_ok = l_run % i_vec == 0;
    // element gathers of this child are repeated for every tile of the other
    // side (128 columns or rows per tile)
    int64_t const l_gathered = l_bytes[l_s] * std::max< int64_t >( 1, l_ext_mn[1 - l_s] / 128 );
    if( l_vec_ok && l_ty == dim_t::K ) l_keep[l_s] = 2;
    else if(    l_vec_ok && l_ty == l_own[l_s]
             && ( l_s == l_col_side ? l_in == l_o_last
                                    : ( l_col_run >= 32 || l_in == l_o_row_last || l_bytes_out < l_bytes[l_s] ) ) ) {
      l_keep[l_s] = 1;
    }
    else if( l_gathered < i_min_bytes_permute ) l_keep[l_s] = 3;
  }
  // one short side (2-64) against a long one: the one-short-side kernel
  // reads the short operand once per workgroup through its offset tables, so
  // a short leaf keeps its layout whatever its gathers (a permute of it is a
  // launch on the tree's path: einsum_benchmark MERA, 1 KB, 5 us), and the
  // long child takes its K order (K stays one affine index in both)
  int64_t const l_short_ext = std::min( l_ext_mn[0], l_ext_mn[1] );
  int const l_short = ( l_ext_mn[0] <= l_ext_mn[1] ) ? 0 : 1;
  // (not with C dims: those nodes can take the tiles, C fastest, whose
  // operand layouts the K order would change; TCCG efbadx,cfx->abcdex 7.7 ->
  // 6.5 TFLOP/s)
  bool const l_has_c = std::find( l_t_out.begin(), l_t_out.end(), dim_t::C ) != l_t_out.end();
  bool const l_skinny_node = !l_has_c && l_short_ext >= 2 && l_short_ext <= 64 && l_ext_mn[1 - l_short] >= 16384;
  if( l_skinny_node && l_fixed[l_short] && l_nd[l_short] > 0 && l_keep[l_short] == 0 ) l_keep[l_short] = 3;
  // two K-read children must agree on the innermost K dim
  if(    l_keep[0] == 2 && l_keep[1] == 2
      && io_dim_ids_left[i_num_dims_left - 1] != io_dim_ids_right[i_num_dims_right - 1] ) {
    l_keep[ l_bytes[0] < l_bytes[1] ? 0 : 1 ] = 0;
  }

  // shared K order: that of a child read along K as it is, else the left's
  int l_k_src = 0;
  if( l_keep[0] != 2 && l_keep[1] == 2 ) l_k_src = 1;
  if( l_skinny_node && l_keep[l_short] != 0 && l_keep[1 - l_short] == 0 ) l_k_src = l_short;
  std::vector< int64_t > l_k_order;
  for( int64_t l_d = 0; l_d < l_nd[l_k_src]; l_d++ ) {
    if( l_t[l_k_src][l_d] == dim_t::K ) l_k_order.push_back( l_ids[l_k_src][l_d] );
  }

  for( int l_s = 0; l_s < 2; l_s++ ) {
    if( l_keep[l_s] != 0 ) continue;
    // the row-side operand M/N-contiguous, the column-side one K-contiguous
    // (the kernel's fastest pairing), unless the extents rule out 16-byte
    // vectors that way
    bool l_mn_inner = ( l_s != l_col_side );
    if( l_mn_inner && l_ext_mn[l_s] % i_vec != 0 && l_ext_k % i_vec == 0 ) l_mn_inner = false;
    if( !l_mn_inner && l_ext_k % i_vec != 0 && l_ext_mn[l_s] % i_vec == 0 ) l_mn_inner = true;
    // neither way gives 16-byte vectors: fp32 takes 8-byte ones along an even
    // run, K first (einsum_benchmark MERA root, M = 3^11, K = 50: 74 us with
    // 8-byte K vectors, 102 with the odd M run gathered; its M = 810, N =
    // 12474, K = 154 node: 47 us either way, 94 gathered)
    if( i_bytes_per_element == 4 && l_ext_mn[l_s] % i_vec != 0 && l_ext_k % i_vec != 0 ) {
      if( l_ext_k % 2 == 0 )              l_mn_inner = false;
      else if( l_ext_mn[l_s] % 2 == 0 )   l_mn_inner = true;
    }
    // one short side (2-64) against a long one: the one-short-side kernel
    // reads the long child coalesced along the long side, so that child takes
    // its own dims innermost, and the node that produces it writes long runs
    // of its output instead of K-length ones (einsum_benchmark MERA: the
    // M = 252, N = 39600 node wrote 6-element runs for its K = 24 consumer)
    if(    std::min( l_ext_mn[0], l_ext_mn[1] ) >= 2 && std::min( l_ext_mn[0], l_ext_mn[1] ) <= 64
        && l_ext_mn[l_s] >= 16384 && l_ext_mn[l_s] > l_ext_mn[1 - l_s] ) {
      l_mn_inner = true;
    }

    std::vector< int64_t > l_c, l_mn, l_x;
    for( dim_t l_ty : { dim_t::C, l_own[l_s] } ) {
      std::vector< int64_t > & l_dst = ( l_ty == dim_t::C ) ? l_c : l_mn;
      for( int64_t l_o = 0; l_o < i_num_dims_out; l_o++ ) {
        if( l_t_out[l_o] != l_ty ) continue;
        for( int64_t l_d = 0; l_d < l_nd[l_s]; l_d++ ) {
          if( l_ids[l_s][l_d] == io_dim_ids_out[l_o] && l_t[l_s][l_d] == l_ty ) {
            l_dst.push_back( l_ids[l_s][l_d] );
            break;
          }
        }
      }
    }
    // dims of this child only (I/J), in their order
    for( int64_t l_d = 0; l_d < l_nd[l_s]; l_d++ ) {
      if( l_t[l_s][l_d] != dim_t::C && l_t[l_s][l_d] != dim_t::K && l_t[l_s][l_d] != l_own[l_s] ) {
        l_x.push_back( l_ids[l_s][l_d] );
      }
    }
    std::vector< int64_t > l_new = l_c;
    l_new.insert( l_new.end(), l_x.begin(), l_x.end() );
    if( l_mn_inner ) {
      l_new.insert( l_new.end(), l_k_order.begin(), l_k_order.end() );
      l_new.insert( l_new.end(), l_mn.begin(), l_mn.end() );
    }
    else {
      l_new.insert( l_new.end(), l_mn.begin(), l_mn.end() );
      l_new.insert( l_new.end(), l_k_order.begin(), l_k_order.end() );
    }
    if( (int64_t) l_new.size() != l_nd[l_s] ) return err_t::DIMENSION_ORDERING_FAILED;
    std::copy( l_new.begin(), l_new.end(), l_ids[l_s] );
  }
  return err_t::SUCCESS;
}

namespace {
  // one tensor walked from its innermost dim outwards: position, dim types
  // and the stride its next dim needs for contiguous storage
  struct BlockCursor {
    int64_t const * ids;
    std::vector< einsum_ir::dim_t > types;
    std::map< int64_t, int64_t > const * strides;
    int64_t pos;
    int64_t cont = 1;

    bool valid() const { return pos >= 0; }
    int64_t id() const { return ids[pos]; }
    einsum_ir::dim_t type() const { return types[pos]; }
    bool contiguous() const { return strides->at( id() ) == cont; }
    void step( int64_t i_size ) { cont *= i_size; pos--; }
  };

  // row-major strides of a dim order
  void default_strides( int64_t i_num_dims, int64_t const * i_ids, std::map< int64_t, int64_t > const * i_sizes,
                        std::map< int64_t, int64_t > & o_strides ) {
    int64_t l_stride = 1;
    for( int64_t l_di = i_num_dims - 1; l_di >= 0; l_di-- ) {
      o_strides[ i_ids[l_di] ] = l_stride;
      l_stride *= i_sizes->at( i_ids[l_di] );
    }
  }

  bool fits( int64_t i_block, int64_t i_size, int64_t i_min, int64_t i_max ) {
    return i_block < i_min || i_block * i_size <= i_max;
  }

  // blocked C dims: trailing output C dims found at the same position (same id,
  // contiguous) in all three tensors.  Returns false when the walk has to stop
  // the whole blocking (a C dim that is not shared contiguously), leaving the
  // collected dims innermost-first as the reference does on that path.
  bool block_c( BlockCursor & io_l, BlockCursor & io_r, BlockCursor & io_o,
                std::map< int64_t, int64_t > const * i_sizes, std::vector< int64_t > & o_cb ) {
    while( io_o.valid() && io_o.type() == einsum_ir::dim_t::C ) {
      if( !io_l.valid() || !io_r.valid() ) return false;
      if( !io_l.contiguous() || !io_r.contiguous() || !io_o.contiguous() ) return false;
      if( io_o.id() != io_l.id() || io_o.id() != io_r.id() ) return false;
      int64_t const l_size = i_sizes->at( io_o.id() );
      o_cb.push_back( io_o.id() );
      io_l.step( l_size );
      io_r.step( l_size );
      io_o.step( l_size );
    }
    return true;
  }

  // blocked dims of one type: the driver tensor's dims of type i_type that sit
  // at the other tensor's cursor too, both contiguous, within the size targets
  void block_pair( einsum_ir::dim_t i_type, BlockCursor & io_drv, BlockCursor & io_other,
                   std::map< int64_t, int64_t > const * i_sizes, int64_t i_min, int64_t i_max,
                   std::vector< int64_t > & o_block ) {
    int64_t l_block = 1;
    while( io_drv.valid() && io_other.valid() && io_drv.type() == i_type ) {
      if( !io_drv.contiguous() || !io_other.contiguous() ) break;
      int64_t const l_size = i_sizes->at( io_drv.id() );
      if( io_drv.id() != io_other.id() || !fits( l_block, l_size, i_min, i_max ) ) break;
      o_block.push_back( io_drv.id() );
      l_block *= l_size;
      io_drv.step( l_size );
      io_other.step( l_size );
    }
  }
}

einsum_ir::err_t einsum_ir::backend::BinaryPrimitives::blocking( primblo_t                            i_primitive_blocking,
                                                                 int64_t                              i_num_dims_left,
                                                                 int64_t                              i_num_dims_right,
                                                                 int64_t                              i_num_dims_out,
                                                                 int64_t                      const * i_dim_ids_left,
                                                                 int64_t                      const * i_dim_ids_right,
                                                                 int64_t                      const * i_dim_ids_out,
                                                                 std::map< int64_t, int64_t > const * i_dim_sizes,
                                                                 std::map< int64_t, int64_t > const * i_strides_left,
                                                                 std::map< int64_t, int64_t > const * i_strides_right,
                                                                 std::map< int64_t, int64_t > const * i_strides_out,
                                                                 std::vector< int64_t >             * o_dim_ids_cb,
                                                                 std::vector< int64_t >             * o_dim_ids_mb,
                                                                 std::vector< int64_t >             * o_dim_ids_nb,
                                                                 std::vector< int64_t >             * o_dim_ids_kb ) const {
  if(    i_primitive_blocking != primblo_t::LEFT_KB_X_MB_CB_RIGHT_NB_X_KB_CB_OUT_NB_X_MB_CB
      && i_primitive_blocking != primblo_t::LEFT_X_CB_KB_MB_RIGHT_X_CB_NB_KB_OUT_NB_X_MB_CB ) {
    return err_t::TENSOR_BLOCKING_FAILED;
  }
  o_dim_ids_cb->clear();
  o_dim_ids_mb->clear();
  o_dim_ids_nb->clear();
  o_dim_ids_kb->clear();

  std::map< int64_t, int64_t > l_def_l, l_def_r, l_def_o;
  if( i_strides_left  == nullptr ) default_strides( i_num_dims_left,  i_dim_ids_left,  i_dim_sizes, l_def_l );
  if( i_strides_right == nullptr ) default_strides( i_num_dims_right, i_dim_ids_right, i_dim_sizes, l_def_r );
  if( i_strides_out   == nullptr ) default_strides( i_num_dims_out,   i_dim_ids_out,   i_dim_sizes, l_def_o );

  BlockCursor l_l{ i_dim_ids_left,  {}, i_strides_left  ? i_strides_left  : &l_def_l, i_num_dims_left  - 1 };
  BlockCursor l_r{ i_dim_ids_right, {}, i_strides_right ? i_strides_right : &l_def_r, i_num_dims_right - 1 };
  BlockCursor l_o{ i_dim_ids_out,   {}, i_strides_out   ? i_strides_out   : &l_def_o, i_num_dims_out   - 1 };
  BinaryContraction::dim_types( i_num_dims_left, i_num_dims_right, i_num_dims_out,
                                i_dim_ids_left, i_dim_ids_right, i_dim_ids_out,
                                &l_l.types, &l_r.types, &l_o.types );
  auto size_at = [&]( BlockCursor const & c ) { return i_dim_sizes->at( c.id() ); };

  if( i_primitive_blocking == primblo_t::LEFT_KB_X_MB_CB_RIGHT_NB_X_KB_CB_OUT_NB_X_MB_CB ) {
    // innermost: C (all three), then M (left/out), K (left/right), N (right/out)
    if( !block_c( l_l, l_r, l_o, i_dim_sizes, *o_dim_ids_cb ) ) return err_t::SUCCESS;
    block_pair( dim_t::M, l_o, l_l, i_dim_sizes, m_size_mb_min, m_size_mb_max, *o_dim_ids_mb );

    // K: continue in the left tensor at the right tensor's next dim, measuring
    // contiguity from that dim's own stride
    int64_t const l_k_id = l_r.valid() ? l_r.id() : 0;
    while( l_l.valid() && !( l_l.type() == dim_t::K && l_l.id() == l_k_id ) ) l_l.step( size_at( l_l ) );
    if( l_l.valid() ) l_l.cont = l_l.strides->at( l_l.id() );
    block_pair( dim_t::K, l_l, l_r, i_dim_sizes, m_size_kb_min, m_size_kb_max, *o_dim_ids_kb );

    // N: the output's next N dim and the same dim in the right tensor
    while( l_o.valid() && l_o.type() != dim_t::N ) l_o.step( size_at( l_o ) );
    int64_t const l_n_id = l_o.valid() ? l_o.id() : 0;
    while( l_r.valid() && !( l_r.type() == dim_t::N && l_r.id() == l_n_id ) ) l_r.step( size_at( l_r ) );
    if( l_r.valid() ) l_r.cont = l_r.strides->at( l_r.id() );
    if( l_o.valid() ) l_o.cont = l_o.strides->at( l_o.id() );
    block_pair( dim_t::N, l_o, l_r, i_dim_sizes, m_size_nb_min, m_size_nb_max, *o_dim_ids_nb );
  }
  else {
    // the inputs' innermost dims (left M then K, right K then N) are not
    // blocked; C is found right behind them
    while( l_l.valid() && l_l.type() == dim_t::M ) l_l.step( size_at( l_l ) );
    while( l_l.valid() && l_l.type() == dim_t::K ) l_l.step( size_at( l_l ) );
    while( l_r.valid() && l_r.type() == dim_t::K ) l_r.step( size_at( l_r ) );
    while( l_r.valid() && l_r.type() == dim_t::N ) l_r.step( size_at( l_r ) );
    if( !block_c( l_l, l_r, l_o, i_dim_sizes, *o_dim_ids_cb ) ) return err_t::SUCCESS;

    // M, K and N from the inputs' innermost dims again
    l_l.pos = i_num_dims_left - 1;
    l_l.cont = 1;
    l_r.pos = i_num_dims_right - 1;
    l_r.cont = 1;
    block_pair( dim_t::M, l_o, l_l, i_dim_sizes, m_size_mb_min, m_size_mb_max, *o_dim_ids_mb );
    block_pair( dim_t::K, l_l, l_r, i_dim_sizes, m_size_kb_min, m_size_kb_max, *o_dim_ids_kb );
    while( l_o.valid() && l_o.type() != dim_t::N ) l_o.pos--;
    if( l_o.valid() ) l_o.cont = l_o.strides->at( l_o.id() );
    block_pair( dim_t::N, l_o, l_r, i_dim_sizes, m_size_nb_min, m_size_nb_max, *o_dim_ids_nb );
  }

  // row-major order
  std::reverse( o_dim_ids_cb->begin(), o_dim_ids_cb->end() );
  std::reverse( o_dim_ids_mb->begin(), o_dim_ids_mb->end() );
  std::reverse( o_dim_ids_nb->begin(), o_dim_ids_nb->end() );
  std::reverse( o_dim_ids_kb->begin(), o_dim_ids_kb->end() );
  return err_t::SUCCESS;
}
