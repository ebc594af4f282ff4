#include "MemoryManager.h"
#include "einsum_ir_hip.h"
#include <algorithm>

einsum_ir::backend::MemoryManager::MemoryManager() : m_alloc( etir_hip_malloc ), m_free( etir_hip_free ) {}

einsum_ir::backend::MemoryManager::~MemoryManager() {
  if( m_arena != nullptr ) {
    m_free( m_arena );
  }
}

int64_t einsum_ir::backend::MemoryManager::reserve_memory( int64_t i_size ) {
  int64_t const l_bytes = ( ( i_size + kGrain - 1 ) / kGrain ) * kGrain;
  int64_t const l_n = ++m_count;
  int64_t l_id;

  if( m_layer_id % 2 == 0 ) {
    int64_t const l_start = edge_of( m_bottom );
    m_place.push_back( l_start );
    m_bottom.push_back( Slot{ l_n, l_start + l_bytes } );
    l_id = l_n;
  }
  else {
    int64_t const l_start = edge_of( m_top ) - l_bytes;
    m_place.push_back( l_start );
    m_top.push_back( Slot{ -l_n, l_start } );
    l_id = -l_n;
  }

  // both stacks together may not overlap: the peak is their combined extent
  m_peak = std::max( m_peak, edge_of( m_bottom ) - edge_of( m_top ) );
  return l_id;
}

void einsum_ir::backend::MemoryManager::remove_reservation( int64_t i_id ) {
  std::vector< Slot > & l_stack = ( i_id >= 0 ) ? m_bottom : m_top;
  auto l_it = std::find_if( l_stack.begin(), l_stack.end(),
                            [i_id]( Slot const & s ) { return s.id == i_id; } );
  if( l_it != l_stack.end() ) l_stack.erase( l_it );
}

einsum_ir::err_t einsum_ir::backend::MemoryManager::alloc_all_memory() {
  if( m_peak <= m_arena_bytes ) return err_t::SUCCESS;
  // a later compile raised the peak: the old arena is too small for the
  // offsets get_mem_ptr now hands out, so it is replaced (nothing in it is
  // live between evaluations)
  if( m_arena != nullptr ) {
    m_free( m_arena );
    m_arena = nullptr;
    m_arena_bytes = 0;
  }
  void * l_ptr = nullptr;
  if( m_alloc( &l_ptr, m_peak ) != 0 || l_ptr == nullptr ) {
    return err_t::UNDEFINED_ERROR;
  }
  m_arena = static_cast< char * >( l_ptr );
  m_arena_bytes = m_peak;
  return err_t::SUCCESS;
}

void * einsum_ir::backend::MemoryManager::get_mem_ptr( int64_t i_id ) {
  if( i_id >= 0 ) {
    return m_arena + m_place[i_id - 1];
  }
  return m_arena + m_peak + m_place[-i_id - 1];
}
