#include "UnaryHip.h"
#include "HostStaging.h"
#include <cstdio>

einsum_ir::backend::UnaryHip::~UnaryHip() {
  if( m_plan != nullptr ) {
    etir_hip_plan_destroy( m_plan );
  }
}

einsum_ir::err_t einsum_ir::backend::UnaryHip::compile() {
  if( compile_base() != err_t::SUCCESS ) {
    return err_t::COMPILATION_FAILED;
  }
  if( m_plan != nullptr ) {
    etir_hip_plan_destroy( m_plan );
    m_plan = nullptr;
  }
  int l_rc = etir_hip_permute_create( m_num_dims, m_sizes_out.data(), m_strides_in.data(),
                                      m_strides_out.data(), m_dtype_in, m_dtype_comp, m_dtype_out,
                                      m_ktype_main, &m_plan );
  if( l_rc != ETIR_SUCCESS ) {
    return static_cast< err_t >( l_rc );
  }
  // bytes spanned by the input and the output: last element offset + 1
  int64_t l_last_in = 0, l_last_out = 0;
  bool l_empty = false;
  for( int64_t l_d = 0; l_d < m_num_dims; l_d++ ) {
    if( m_sizes_out[l_d] <= 0 ) l_empty = true;
    l_last_in  += ( m_sizes_out[l_d] - 1 ) * m_strides_in[l_d];
    l_last_out += ( m_sizes_out[l_d] - 1 ) * m_strides_out[l_d];
  }
  m_bytes_in  = l_empty ? 0 : ( l_last_in + 1 ) * ce_n_bytes( m_dtype_in );
  m_bytes_out = l_empty ? 0 : ( l_last_out + 1 ) * ce_n_bytes( m_dtype_out );
  m_compiled = true;
  return err_t::SUCCESS;
}

einsum_ir::err_t einsum_ir::backend::UnaryHip::eval_async( void const * i_tensor_in,
                                                           void       * io_tensor_out ) {
  if( !m_compiled ) {
    return err_t::CALLED_BEFORE_COMPILATION;
  }
  return static_cast< err_t >( etir_hip_permute_execute( m_plan, i_tensor_in, io_tensor_out, m_stream ) );
}

void einsum_ir::backend::UnaryHip::eval( void const * i_tensor_in,
                                         void       * io_tensor_out ) {
  if( !m_compiled ) {
    m_last_error = err_t::CALLED_BEFORE_COMPILATION;
  }
  else {
    // host tensors go through device copies; the output is copied in too
    // (ADD reads it, and elements outside the permuted view keep their values)
    HostStaging l_st;
    void const * l_in  = l_st.stage( i_tensor_in,   m_bytes_in,  true, false );
    void       * l_out = l_st.stage( io_tensor_out, m_bytes_out, true, true );
    m_last_error = l_st.error();
    if( m_last_error == err_t::SUCCESS ) m_last_error = eval_async( l_in, l_out );
    if( m_last_error == err_t::SUCCESS && etir_hip_synchronize( m_stream ) != ETIR_SUCCESS ) {
      m_last_error = err_t::UNDEFINED_ERROR;
    }
    if( m_last_error == err_t::SUCCESS && l_st.active() ) m_last_error = l_st.finish();
  }
  if( m_last_error != err_t::SUCCESS ) {
    std::fprintf( stderr, "einsum_ir: permutation failed (%d): %s\n", (int) m_last_error,
                  etir_hip_last_error() );
  }
}
