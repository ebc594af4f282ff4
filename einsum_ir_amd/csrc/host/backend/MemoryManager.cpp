#include "MemoryManager.h"
#include "einsum_ir_hip.h"
#include <algorithm>

einsum_ir::backend::MemoryManager::~MemoryManager() {
  if( m_memory_ptr != nullptr ) {
    etir_hip_free( m_memory_ptr );
  }
}

int64_t einsum_ir::backend::MemoryManager::reserve_memory( int64_t i_size ) {
  m_last_id++;
  if( i_size % m_alignment != 0 ) {
    i_size += m_alignment - ( i_size % m_alignment );
  }

  int64_t l_id = 0;
  int64_t l_offset = 0;
  if( m_layer_id % 2 == 0 ) {
    // left stack grows upwards from 0
    if( !m_allocated_offset_left.empty() ) l_offset = m_allocated_offset_left.front();
    m_tensor_offset.push_back( l_offset );
    l_id = m_last_id;
    m_allocated_id_left.push_front( l_id );
    m_allocated_offset_left.push_front( l_offset + i_size );
  }
  else {
    // right stack grows downwards from the end
    if( !m_allocated_offset_right.empty() ) l_offset = m_allocated_offset_right.front();
    l_offset -= i_size;
    m_tensor_offset.push_back( l_offset );
    l_id = -m_last_id;
    m_allocated_id_right.push_front( l_id );
    m_allocated_offset_right.push_front( l_offset );
  }

  int64_t l_top_left  = m_allocated_offset_left.empty()  ? 0 : m_allocated_offset_left.front();
  int64_t l_top_right = m_allocated_offset_right.empty() ? 0 : m_allocated_offset_right.front();
  m_req_mem = std::max( m_req_mem, l_top_left - l_top_right );
  return l_id;
}

void einsum_ir::backend::MemoryManager::remove_reservation( int64_t i_id ) {
  std::list< int64_t > & l_ids  = ( i_id >= 0 ) ? m_allocated_id_left     : m_allocated_id_right;
  std::list< int64_t > & l_offs = ( i_id >= 0 ) ? m_allocated_offset_left : m_allocated_offset_right;
  auto l_it_off = l_offs.begin();
  for( auto l_it = l_ids.begin(); l_it != l_ids.end(); ++l_it, ++l_it_off ) {
    if( *l_it == i_id ) {
      l_ids.erase( l_it );
      l_offs.erase( l_it_off );
      return;
    }
  }
}

einsum_ir::err_t einsum_ir::backend::MemoryManager::alloc_all_memory() {
  if( m_req_mem > 0 && m_memory_ptr == nullptr ) {
    void * l_ptr = nullptr;
    if( etir_hip_malloc( &l_ptr, m_req_mem ) != 0 ) {
      return err_t::UNDEFINED_ERROR;
    }
    m_memory_ptr = static_cast< char * >( l_ptr );
  }
  return err_t::SUCCESS;
}

void * einsum_ir::backend::MemoryManager::get_mem_ptr( int64_t i_id ) {
  if( i_id >= 0 ) {
    return m_memory_ptr + m_tensor_offset[i_id - 1];
  }
  return m_memory_ptr + m_req_mem + m_tensor_offset[-i_id - 1];
}
