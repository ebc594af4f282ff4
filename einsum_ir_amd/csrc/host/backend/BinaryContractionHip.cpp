#include <stdexcept>
#include "BinaryContractionHip.h"
#include "HostStaging.h"
#include "Tensor.h"
#include <cstdio>

einsum_ir::backend::BinaryContractionHip::~BinaryContractionHip() {
  if( m_plan != nullptr ) {
    etir_hip_plan_destroy( m_plan );
  }
}

einsum_ir::err_t einsum_ir::backend::BinaryContractionHip::compile() {
  err_t l_err = compile_base();
  if( l_err != err_t::SUCCESS ) {
    return l_err;
  }
  if( m_dim_sizes_outer_left == nullptr || m_dim_sizes_outer_right == nullptr
      || m_dim_sizes_outer_out == nullptr ) {
    return err_t::COMPILATION_FAILED;
  }

  // element strides of every tensor keyed by dim id
  std::map< int64_t, int64_t > l_s_left, l_s_right, l_s_out, l_s_aux;
  try {
    strides( m_num_dims_left,  m_dim_ids_left,  m_dim_sizes_outer_left,  &l_s_left );
    strides( m_num_dims_right, m_dim_ids_right, m_dim_sizes_outer_right, &l_s_right );
    strides( m_num_dims_out,   m_dim_ids_out,   m_dim_sizes_outer_out,   &l_s_out );
    // the auxiliary tensor has its own outer sizes; without them it shares the
    // output's layout for COPY/ADD first touches and is a scalar otherwise
    // (reference BinaryContractionTpp.cpp:31-41)
    if( m_dim_sizes_outer_out_aux != nullptr ) {
      strides( m_num_dims_out, m_dim_ids_out, m_dim_sizes_outer_out_aux, &l_s_aux );
    }
    else if( m_ktype_first_touch == kernel_t::ADD || m_ktype_first_touch == kernel_t::COPY ) {
      l_s_aux = l_s_out;
    }
  }
  catch( std::out_of_range const & ) {
    return err_t::COMPILATION_FAILED;
  }

  // tensor sizes in bytes (for staging host tensors in contract())
  try {
    int64_t const l_esz_out = ce_n_bytes( m_dtype_out );
    m_bytes[0] = Tensor::size( ce_n_bytes( m_dtype_left ), m_num_dims_left, m_dim_ids_left, *m_dim_sizes_outer_left );
    m_bytes[1] = Tensor::size( ce_n_bytes( m_dtype_right ), m_num_dims_right, m_dim_ids_right, *m_dim_sizes_outer_right );
    m_bytes[3] = Tensor::size( l_esz_out, m_num_dims_out, m_dim_ids_out, *m_dim_sizes_outer_out );
    m_bytes[2] = ( m_dim_sizes_outer_out_aux != nullptr )
               ? Tensor::size( l_esz_out, m_num_dims_out, m_dim_ids_out, *m_dim_sizes_outer_out_aux )
               : ( l_s_aux.empty() ? l_esz_out : m_bytes[3] );
  }
  catch( std::out_of_range const & ) {
    return err_t::COMPILATION_FAILED;
  }

  auto find0 = []( std::map< int64_t, int64_t > const & i_map, int64_t i_key ) -> int64_t {
    auto l_it = i_map.find( i_key );
    return l_it == i_map.end() ? 0 : l_it->second;
  };

  // one loop per C, M, N, K dim (reference BinaryContractionTpp.cpp:46-66)
  std::vector< int64_t > l_ids;
  l_ids.insert( l_ids.end(), m_dim_ids_c.begin(), m_dim_ids_c.end() );
  l_ids.insert( l_ids.end(), m_dim_ids_m.begin(), m_dim_ids_m.end() );
  l_ids.insert( l_ids.end(), m_dim_ids_n.begin(), m_dim_ids_n.end() );
  l_ids.insert( l_ids.end(), m_dim_ids_k.begin(), m_dim_ids_k.end() );
  std::size_t const l_n = l_ids.size();
  std::vector< int32_t > l_types( l_n );
  std::vector< int64_t > l_sizes( l_n ), l_sl( l_n ), l_sr( l_n ), l_sa( l_n ), l_so( l_n );
  for( std::size_t l_i = 0; l_i < l_n; l_i++ ) {
    int64_t const l_id = l_ids[l_i];
    l_types[l_i] = (int32_t) m_dim_types.at( l_id );
    l_sizes[l_i] = m_dim_sizes_inner->at( l_id );
    l_sl[l_i] = find0( l_s_left,  l_id );
    l_sr[l_i] = find0( l_s_right, l_id );
    l_sa[l_i] = find0( l_s_aux,   l_id );
    l_so[l_i] = find0( l_s_out,   l_id );
  }

  // complex kernels: one C dim is the complex dim
  if( m_ktype_main == kernel_t::CPX_MADD ) {
    int64_t const l_cpx = ( m_cpx_dim_id >= 0 ) ? m_cpx_dim_id
                        : ( m_dim_ids_c.empty() ? -1 : m_dim_ids_c[0] );
    std::size_t l_i = 0;
    while( l_i < l_n && !( l_ids[l_i] == l_cpx && l_types[l_i] == (int32_t) dim_t::C ) ) l_i++;
    if( l_i == l_n || l_sizes[l_i] != 2 ) return err_t::INVALID_CPX_DIM;
    l_types[l_i] = (int32_t) dim_t::CPX;
  }

  if( m_plan != nullptr ) {
    etir_hip_plan_destroy( m_plan );
    m_plan = nullptr;
  }
  int l_rc = etir_hip_contraction_create( (int64_t) l_n, l_types.data(), l_sizes.data(),
                                          l_sl.data(), l_sr.data(), l_sa.data(), l_so.data(),
                                          m_dtype_left, m_dtype_right, m_dtype_comp, m_dtype_out,
                                          m_ktype_first_touch, m_ktype_main, m_ktype_last_touch,
                                          &m_plan );
  if( l_rc != ETIR_SUCCESS ) {
    return static_cast< err_t >( l_rc );
  }
  m_compiled = true;
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::BinaryContractionHip::contract_async( void const * i_tensor_left,
                                                                           void const * i_tensor_right,
                                                                           void const * i_tensor_out_aux,
                                                                           void       * io_tensor_out ) {
  if( !m_compiled ) {
    return err_t::CALLED_BEFORE_COMPILATION;
  }
  int l_rc = etir_hip_contraction_execute( m_plan, i_tensor_left, i_tensor_right,
                                           i_tensor_out_aux, io_tensor_out, m_stream );
  return static_cast< err_t >( l_rc );
}

void einsum_ir::backend::BinaryContractionHip::contract( void const * i_tensor_left,
                                                         void const * i_tensor_right,
                                                         void       * io_tensor_out ) {
  contract( i_tensor_left, i_tensor_right, nullptr, io_tensor_out );
}

void einsum_ir::backend::BinaryContractionHip::contract( void const * i_tensor_left,
                                                         void const * i_tensor_right,
                                                         void const * i_tensor_out_aux,
                                                         void       * io_tensor_out ) {
  if( !m_compiled ) {
    m_last_error = err_t::CALLED_BEFORE_COMPILATION;
  }
  else {
    // host tensors (the reference's callers pass them) go through device copies
    HostStaging l_st;
    void const * l_left  = l_st.stage( i_tensor_left,    m_bytes[0], true, false );
    void const * l_right = l_st.stage( i_tensor_right,   m_bytes[1], true, false );
    void const * l_aux   = l_st.stage( i_tensor_out_aux, m_bytes[2], true, false );
    void       * l_out   = l_st.stage( io_tensor_out,    m_bytes[3], true, true );
    m_last_error = l_st.error();
    if( m_last_error == err_t::SUCCESS ) {
      m_last_error = contract_async( l_left, l_right, l_aux, l_out );
    }
    if( m_last_error == err_t::SUCCESS && etir_hip_synchronize( m_stream ) != ETIR_SUCCESS ) {
      m_last_error = err_t::UNDEFINED_ERROR;
    }
    if( m_last_error == err_t::SUCCESS && l_st.active() ) {
      m_last_error = l_st.finish();
    }
  }
  if( m_last_error != err_t::SUCCESS ) {
    std::fprintf( stderr, "einsum_ir: contraction failed (%d): %s\n", (int) m_last_error,
                  etir_hip_last_error() );
  }
}
