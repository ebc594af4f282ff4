// Arena for the intermediate tensors of an einsum tree, placed in HBM.
//
// Same planning interface as the reference's MemoryManager
// (reference src/backend/MemoryManager.h:15-90): reservations of even tree
// layers are stacked upwards from the bottom of the arena and those of odd
// layers downwards from its top (reference src/backend/MemoryManager.cpp:9-79),
// so a parent's output and its children's outputs never overlap while both
// are live.  alloc_all_memory() makes ONE device allocation (etir_hip_malloc)
// for the planned peak, and makes a new, larger one when a later compile on
// the same manager raises the peak; get_mem_ptr() returns device pointers
// into the current allocation.
#ifndef EINSUM_IR_BACKEND_MEMORY_MANAGER
#define EINSUM_IR_BACKEND_MEMORY_MANAGER

#include <cstdint>
#include <vector>
#include "../constants.h"

namespace einsum_ir {
  namespace backend {
    class MemoryManager;
  }
}

class einsum_ir::backend::MemoryManager {
  private:
    //! reservations are rounded up to this many bytes (keeps 256-byte device alignment)
    static constexpr int64_t kGrain = 256;

    //! a live reservation on one of the two stacks: its id and the edge it
    //! leaves for the next reservation on that stack (bottom stack: its end
    //! offset; top stack: its start offset, negative, relative to the peak)
    struct Slot {
      int64_t id;
      int64_t edge;
    };

    //! allocator of the arena (device memory unless a caller swaps it)
    int  ( *m_alloc )( void **, int64_t ) = nullptr;
    int  ( *m_free  )( void * )           = nullptr;

    char *  m_arena       = nullptr;   //!< device allocation
    int64_t m_arena_bytes = 0;         //!< its size
    int64_t m_peak        = 0;         //!< planned peak (bytes)
    int64_t m_count       = 0;         //!< reservations made so far

    //! placement of reservation n (index n - 1); top-stack placements are
    //! negative offsets from the peak
    std::vector< int64_t > m_place;

    std::vector< Slot > m_bottom;      //!< back() = most recent live reservation
    std::vector< Slot > m_top;

    static int64_t edge_of( std::vector< Slot > const & i_stack ) {
      return i_stack.empty() ? 0 : i_stack.back().edge;
    }

  public:
    //! layer of the tree that is currently being planned
    int64_t m_layer_id = 0;

    MemoryManager();
    MemoryManager( MemoryManager const & ) = delete;
    MemoryManager & operator=( MemoryManager const & ) = delete;
    ~MemoryManager();

    /** Plans a reservation of i_size bytes; returns its id (> 0 bottom stack, < 0 top stack). **/
    int64_t reserve_memory( int64_t i_size );

    /** Ends the lifetime of a reservation (planning only). **/
    void remove_reservation( int64_t i_id );

    /** Makes sure the device arena holds the planned peak (allocates or grows it). **/
    err_t alloc_all_memory();

    /** Device pointer of a reservation. **/
    void * get_mem_ptr( int64_t i_id );

    /** Peak bytes of the plan. **/
    int64_t get_required_memory() const { return m_peak; }

    /** Replaces the arena allocator (etir_hip_malloc / etir_hip_free by default);
        only before the first alloc_all_memory. **/
    void set_allocator( int ( *i_alloc )( void **, int64_t ), int ( *i_free )( void * ) ) {
      m_alloc = i_alloc;
      m_free  = i_free;
    }

    /** Takes the allocator of another manager (an arena planned beside it). **/
    void share_allocator( MemoryManager const & i_other ) {
      m_alloc = i_other.m_alloc;
      m_free  = i_other.m_free;
    }

    /** Bytes of the current device allocation (0 before alloc_all_memory). **/
    int64_t get_allocated_memory() const { return m_arena_bytes; }
};

#endif
