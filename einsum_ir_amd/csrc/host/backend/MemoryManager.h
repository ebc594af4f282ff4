// Arena for the intermediate tensors of an einsum tree, placed in HBM.
//
// Same planning interface as the reference's MemoryManager
// (reference src/backend/MemoryManager.h:15-90): a two-sided stack where
// reservations of even tree layers grow from the left end and odd layers from
// the right end (reference src/backend/MemoryManager.cpp:9-79), so a parent's
// output and its children's outputs never overlap while both are live.
// alloc_all_memory() makes ONE device allocation (etir_hip_malloc) for the
// peak requirement; get_mem_ptr() returns device pointers.
#ifndef EINSUM_IR_BACKEND_MEMORY_MANAGER
#define EINSUM_IR_BACKEND_MEMORY_MANAGER

#include <cstdint>
#include <list>
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
    int64_t m_alignment = 256;

    char * m_memory_ptr = nullptr;
    int64_t m_req_mem = 0;
    int64_t m_last_id = 0;

    //! offset of every reservation (index id-1); right-side offsets are negative
    std::vector< int64_t > m_tensor_offset;

    //! live reservations on both sides (front = top of the stack)
    std::list< int64_t > m_allocated_id_left;
    std::list< int64_t > m_allocated_id_right;
    std::list< int64_t > m_allocated_offset_left;
    std::list< int64_t > m_allocated_offset_right;

  public:
    //! layer of the tree that is currently being planned
    int64_t m_layer_id = 0;

    ~MemoryManager();

    /** Plans a reservation of i_size bytes; returns its id (> 0 left side, < 0 right side). **/
    int64_t reserve_memory( int64_t i_size );

    /** Ends the lifetime of a reservation (planning only). **/
    void remove_reservation( int64_t i_id );

    /** Allocates the device arena for the planned peak. **/
    err_t alloc_all_memory();

    /** Device pointer of a reservation. **/
    void * get_mem_ptr( int64_t i_id );

    /** Peak bytes of the plan. **/
    int64_t get_required_memory() const { return m_req_mem; }
};

#endif
