// Device copies of tensors that live in pageable host memory.
//
// The reference's operators take host tensors (at::Tensor CPU data, reference
// src/bench_binary.cpp:132-134); the HIP kernels need memory the GPU can
// reach.  The synchronous operator calls (BinaryContractionHip::contract,
// UnaryHip::eval, EinsumNode::eval / store_and_lock_data) pass every tensor
// pointer through stage(): GPU-accessible pointers come back unchanged, host
// ones are replaced by a device copy (filled from the host when the call
// reads the tensor) that finish() copies back when the call writes it.  The
// asynchronous calls take device pointers only.
#ifndef EINSUM_IR_BACKEND_HOST_STAGING
#define EINSUM_IR_BACKEND_HOST_STAGING

#include <cstdint>
#include <vector>
#include "../constants.h"

namespace einsum_ir {
  namespace backend {
    class HostStaging;
  }
}

class einsum_ir::backend::HostStaging {
  private:
    struct Entry {
      void    * host;
      void    * dev;
      int64_t   bytes;
      bool      copy_back;
    };
    std::vector< Entry > m_entries;
    err_t m_err = err_t::SUCCESS;

  public:
    HostStaging() = default;
    HostStaging( HostStaging const & ) = delete;
    HostStaging & operator=( HostStaging const & ) = delete;

    //! frees the device copies (without copying back)
    ~HostStaging();

    /**
     * Returns a pointer the GPU can access for i_ptr (i_bytes bytes): i_ptr
     * itself, an earlier copy of the same host pointer, or a new device copy
     * (copied from the host if i_copy_in).  i_copy_back marks the copy to be
     * written back by finish().  nullptr stays nullptr.  On failure returns
     * nullptr and error() is set.
     **/
    void * stage( void const * i_ptr,
                  int64_t      i_bytes,
                  bool         i_copy_in,
                  bool         i_copy_back );

    //! true if at least one tensor was copied
    bool active() const { return !m_entries.empty(); }

    //! copies the written tensors back to the host (after the device work
    //! finished: the caller synchronises first)
    err_t finish();

    err_t error() const { return m_err; }
};

#endif
