// Backend registry for binary contractions (reference
// src/backend/BinaryContractionFactory.{h,cpp}:17-67).  This library is built
// for the MI355X only: HIP is the one supported backend; AUTO resolves to it
// in EinsumNode.  Other backend values are reported as unsupported.
#ifndef EINSUM_IR_BACKEND_BINARY_CONTRACTION_FACTORY
#define EINSUM_IR_BACKEND_BINARY_CONTRACTION_FACTORY

#include "BinaryContraction.h"

namespace einsum_ir {
  namespace backend {
    class BinaryContractionFactory;
  }
}

class einsum_ir::backend::BinaryContractionFactory {
  public:
    static bool supports( backend_t i_backend );
    static BinaryContraction * create( backend_t i_backend );
};

#endif
