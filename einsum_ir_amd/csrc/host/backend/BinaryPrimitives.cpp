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
  tenord_t l_ord = tenord_t::LEFT_NATIVE_RIGHT_NATIVE_OUT_NATIVE;
  if( i_backend_type == backend_t::TPP || i_backend_type == backend_t::TBLIS || i_backend_type == backend_t::HIP ) {
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
