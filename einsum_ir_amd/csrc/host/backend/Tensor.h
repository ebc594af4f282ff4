// Byte size of a tensor from its dimension ids and sizes
// (reference src/backend/Tensor.h / Tensor.cpp:5-15).
#ifndef EINSUM_IR_BACKEND_TENSOR
#define EINSUM_IR_BACKEND_TENSOR

#include <cstdint>
#include <map>

namespace einsum_ir {
  namespace backend {
    class Tensor;
  }
}

class einsum_ir::backend::Tensor {
  public:
    static int64_t size( int64_t                              i_bytes_per_entry,
                         int64_t                              i_num_dims,
                         int64_t                      const * i_dim_ids,
                         std::map< int64_t, int64_t > const & i_dim_sizes );
};

#endif
