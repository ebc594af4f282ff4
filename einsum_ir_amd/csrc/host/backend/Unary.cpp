#include <stdexcept>
#include "Unary.h"

void einsum_ir::backend::Unary::strides( int64_t                              i_num_dims,
                                         std::map< int64_t, int64_t > const * i_dim_sizes,
                                         int64_t                      const * i_dim_ids,
                                         int64_t                            * o_strides ) {
  int64_t l_stride = 1;
  for( int64_t l_di = i_num_dims - 1; l_di >= 0; l_di-- ) {
    o_strides[l_di] = l_stride;
    l_stride *= i_dim_sizes->at( i_dim_ids[l_di] );
  }
}

void einsum_ir::backend::Unary::order_strides_output_based( int64_t         i_num_dims,
                                                            int64_t const * i_dim_ids_in,
                                                            int64_t const * i_dim_ids_out,
                                                            int64_t       * io_strides ) {
  std::map< int64_t, int64_t > l_by_id;
  for( int64_t l_di = 0; l_di < i_num_dims; l_di++ ) {
    l_by_id.insert( { i_dim_ids_in[l_di], io_strides[l_di] } );
  }
  for( int64_t l_di = 0; l_di < i_num_dims; l_di++ ) {
    io_strides[l_di] = l_by_id.at( i_dim_ids_out[l_di] );
  }
}

void einsum_ir::backend::Unary::init( int64_t                              i_num_dims,
                                      std::map< int64_t, int64_t > const * i_dim_sizes,
                                      int64_t                      const * i_dim_ids_in,
                                      int64_t                      const * i_dim_ids_out,
                                      data_t                               i_dtype_in,
                                      data_t                               i_dtype_comp,
                                      data_t                               i_dtype_out,
                                      kernel_t                             i_ktype_main,
                                      int64_t                              i_num_threads ) {
  init( i_num_dims, i_dim_sizes, i_dim_ids_in, i_dim_ids_out, nullptr, nullptr,
        i_dtype_in, i_dtype_comp, i_dtype_out, i_ktype_main, i_num_threads );
}

void einsum_ir::backend::Unary::init( int64_t                              i_num_dims,
                                      std::map< int64_t, int64_t > const * i_dim_sizes,
                                      int64_t                      const * i_dim_ids_in,
                                      int64_t                      const * i_dim_ids_out,
                                      int64_t                            * i_strides_in,
                                      int64_t                            * i_strides_out,
                                      data_t                               i_dtype_in,
                                      data_t                               i_dtype_comp,
                                      data_t                               i_dtype_out,
                                      kernel_t                             i_ktype_main,
                                      int64_t                              i_num_threads ) {
  m_num_dims    = i_num_dims;
  m_dim_sizes   = i_dim_sizes;
  m_dim_ids_in  = i_dim_ids_in;
  m_dim_ids_out = i_dim_ids_out;
  m_dtype_in    = i_dtype_in;
  m_dtype_comp  = i_dtype_comp;
  m_dtype_out   = i_dtype_out;
  m_ktype_main  = i_ktype_main;
  m_num_threads = i_num_threads;
  m_strides_in.clear();
  m_strides_out.clear();
  if( i_strides_in != nullptr )  m_strides_in.assign( i_strides_in, i_strides_in + i_num_dims );
  if( i_strides_out != nullptr ) m_strides_out.assign( i_strides_out, i_strides_out + i_num_dims );
}

einsum_ir::err_t einsum_ir::backend::Unary::compile_base() {
  try {
    m_sizes_out.resize( m_num_dims );
    for( int64_t l_di = 0; l_di < m_num_dims; l_di++ ) {
      m_sizes_out[l_di] = m_dim_sizes->at( m_dim_ids_out[l_di] );
    }
    if( m_strides_in.empty() ) {
      m_strides_in.resize( m_num_dims );
      strides( m_num_dims, m_dim_sizes, m_dim_ids_in, m_strides_in.data() );
    }
    if( m_strides_out.empty() ) {
      m_strides_out.resize( m_num_dims );
      strides( m_num_dims, m_dim_sizes, m_dim_ids_out, m_strides_out.data() );
    }
    order_strides_output_based( m_num_dims, m_dim_ids_in, m_dim_ids_out, m_strides_in.data() );
  }
  catch( std::out_of_range const & ) {
    return err_t::COMPILATION_FAILED;
  }
  return err_t::SUCCESS;
}
