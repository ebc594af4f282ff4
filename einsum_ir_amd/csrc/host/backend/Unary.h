// Unary (permutation) operator base class, drop-in for the reference's
// einsum_ir::backend::Unary (reference src/backend/Unary.h:15-158).
#ifndef EINSUM_IR_BACKEND_UNARY
#define EINSUM_IR_BACKEND_UNARY

#include <cstdint>
#include <map>
#include <vector>
#include "../constants.h"

namespace einsum_ir {
  namespace backend {
    class Unary;
  }
}

class einsum_ir::backend::Unary {
  public:
    int64_t m_num_dims = 0;
    std::map< int64_t, int64_t > const * m_dim_sizes = nullptr;
    int64_t const * m_dim_ids_in = nullptr;
    int64_t const * m_dim_ids_out = nullptr;

    //! sizes in output order
    std::vector< int64_t > m_sizes_out;
    //! input strides in output-dimension order
    std::vector< int64_t > m_strides_in;
    //! output strides
    std::vector< int64_t > m_strides_out;

    data_t m_dtype_in = UNDEFINED_DTYPE;
    data_t m_dtype_comp = UNDEFINED_DTYPE;
    data_t m_dtype_out = UNDEFINED_DTYPE;
    kernel_t m_ktype_main = UNDEFINED_KTYPE;
    int64_t m_num_threads = 1;

    /** Row-major strides of a tensor (position-indexed, reference Unary.cpp:3-14). **/
    static void strides( int64_t                              i_num_dims,
                         std::map< int64_t, int64_t > const * i_dim_sizes,
                         int64_t                      const * i_dim_ids,
                         int64_t                            * o_strides );

    /** Reorders input strides into the output's dim order (reference Unary.cpp:16-31). **/
    static void order_strides_output_based( int64_t         i_num_dims,
                                            int64_t const * i_dim_ids_in,
                                            int64_t const * i_dim_ids_out,
                                            int64_t       * io_strides );

    virtual ~Unary() {}

    void init( int64_t                              i_num_dims,
               std::map< int64_t, int64_t > const * i_dim_sizes,
               int64_t                      const * i_dim_ids_in,
               int64_t                      const * i_dim_ids_out,
               data_t                               i_dtype_in,
               data_t                               i_dtype_comp,
               data_t                               i_dtype_out,
               kernel_t                             i_ktype_main,
               int64_t                              i_num_threads );

    void init( int64_t                              i_num_dims,
               std::map< int64_t, int64_t > const * i_dim_sizes,
               int64_t                      const * i_dim_ids_in,
               int64_t                      const * i_dim_ids_out,
               int64_t                            * i_strides_in,
               int64_t                            * i_strides_out,
               data_t                               i_dtype_in,
               data_t                               i_dtype_comp,
               data_t                               i_dtype_out,
               kernel_t                             i_ktype_main,
               int64_t                              i_num_threads );

    /** Sizes in output order; strides (derived unless given); input strides reordered. **/
    err_t compile_base();

    virtual err_t compile() = 0;

    virtual void eval( void const * i_tensor_in,
                       void       * io_tensor_out ) = 0;
};

#endif
