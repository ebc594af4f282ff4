// BinaryContraction on the MI355X: compile() lowers the contraction to the
// loop IR and creates one device plan through the C ABI
// (etir_hip_contraction_create); contract() launches it.
//
// Sibling of the reference's BinaryContractionTpp
// (reference src/backend/BinaryContractionTpp.{h,cpp}); the lowering follows
// BinaryContractionTpp::compile (reference src/backend/BinaryContractionTpp.cpp:4-127).
// contract() is synchronous like the reference's and accepts host tensors
// too (staged through device copies, HostStaging.h); contract_async() only
// enqueues on the plan's stream and takes device pointers (used by EinsumNode
// to run a whole tree on one stream).
#ifndef EINSUM_IR_BACKEND_BINARY_CONTRACTION_HIP
#define EINSUM_IR_BACKEND_BINARY_CONTRACTION_HIP

#include "BinaryContraction.h"
#include "einsum_ir_hip.h"

namespace einsum_ir {
  namespace backend {
    class BinaryContractionHip;
  }
}

class einsum_ir::backend::BinaryContractionHip : public BinaryContraction {
  private:
    etir_plan_t m_plan = nullptr;
    void * m_stream = nullptr;
    err_t m_last_error = err_t::SUCCESS;
    //! bytes of the left, right, auxiliary and output tensors (outer sizes)
    int64_t m_bytes[4] = { 0, 0, 0, 0 };

  public:
    ~BinaryContractionHip();

    err_t compile();

    /** Selects the HIP stream (hipStream_t as void*, nullptr = null stream). **/
    void set_stream( void * i_stream ) { m_stream = i_stream; }

    //! complex kernels: id of the complex dim (size 2); -1 selects the first
    //! C dim in the output's order, the reference BLAS backend's rule
    //! (reference src/backend/BinaryContractionBlas.cpp:82-85)
    int64_t m_cpx_dim_id = -1;

    void contract( void const * i_tensor_left,
                   void const * i_tensor_right,
                   void       * io_tensor_out );

    void contract( void const * i_tensor_left,
                   void const * i_tensor_right,
                   void const * i_tensor_out_aux,
                   void       * io_tensor_out );

    /** Enqueues the contraction on the stream without waiting. **/
    err_t contract_async( void const * i_tensor_left,
                          void const * i_tensor_right,
                          void const * i_tensor_out_aux,
                          void       * io_tensor_out );

    /** Error of the last contract() call (contract() itself returns void). **/
    err_t last_error() const { return m_last_error; }

    /** The device plan (diagnostics: etir_hip_plan_describe). **/
    etir_plan_t plan() const { return m_plan; }
};

#endif
