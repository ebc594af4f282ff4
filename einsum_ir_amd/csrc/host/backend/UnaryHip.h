// Unary operator on the MI355X: one device permutation plan per operator
// (etir_hip_permute_create), sibling of the reference's UnaryTpp
// (reference src/backend/UnaryTpp.cpp:4-54).  eval() is synchronous and
// accepts host tensors too (staged through device copies, HostStaging.h);
// eval_async() only enqueues on the stream and takes device pointers.
#ifndef EINSUM_IR_BACKEND_UNARY_HIP
#define EINSUM_IR_BACKEND_UNARY_HIP

#include "Unary.h"
#include "einsum_ir_hip.h"

namespace einsum_ir {
  namespace backend {
    class UnaryHip;
  }
}

class einsum_ir::backend::UnaryHip : public Unary {
  private:
    etir_plan_t m_plan = nullptr;
    void * m_stream = nullptr;
    bool m_compiled = false;
    err_t m_last_error = err_t::SUCCESS;
    //! bytes spanned by the input and the output (for staging host tensors)
    int64_t m_bytes_in = 0;
    int64_t m_bytes_out = 0;

  public:
    ~UnaryHip();

    err_t compile();

    void set_stream( void * i_stream ) { m_stream = i_stream; }

    void eval( void const * i_tensor_in,
               void       * io_tensor_out );

    err_t eval_async( void const * i_tensor_in,
                      void       * io_tensor_out );

    err_t last_error() const { return m_last_error; }

    etir_plan_t plan() const { return m_plan; }
};

#endif
