#include "HostStaging.h"
#include "einsum_ir_hip.h"

einsum_ir::backend::HostStaging::~HostStaging() {
  for( Entry const & l_e : m_entries ) etir_hip_free( l_e.dev );
}

void * einsum_ir::backend::HostStaging::stage( void const * i_ptr,
                                               int64_t      i_bytes,
                                               bool         i_copy_in,
                                               bool         i_copy_back ) {
  if( i_ptr == nullptr ) return nullptr;
  if( etir_hip_pointer_is_device( i_ptr ) == 1 ) return const_cast< void * >( i_ptr );
  for( Entry & l_e : m_entries ) {
    if( l_e.host == i_ptr ) {
      l_e.copy_back = l_e.copy_back || i_copy_back;
      return l_e.dev;
    }
  }
  void * l_dev = nullptr;
  if( i_bytes <= 0 || etir_hip_malloc( &l_dev, i_bytes ) != ETIR_SUCCESS ) {
    m_err = err_t::UNDEFINED_ERROR;
    return nullptr;
  }
  m_entries.push_back( Entry{ const_cast< void * >( i_ptr ), l_dev, i_bytes, i_copy_back } );
  if( i_copy_in && etir_hip_memcpy_h2d( l_dev, i_ptr, i_bytes ) != ETIR_SUCCESS ) {
    m_err = err_t::UNDEFINED_ERROR;
    return nullptr;
  }
  return l_dev;
}

einsum_ir::err_t einsum_ir::backend::HostStaging::finish() {
  for( Entry const & l_e : m_entries ) {
    if( l_e.copy_back && etir_hip_memcpy_d2h( l_e.host, l_e.dev, l_e.bytes ) != ETIR_SUCCESS ) {
      m_err = err_t::UNDEFINED_ERROR;
    }
  }
  return m_err;
}
