// Binary contraction operator base class (drop-in for the reference's
// einsum_ir::backend::BinaryContraction, reference src/backend/BinaryContraction.h:16-393).
//
// Same public members, same two init overloads, same pure virtual
// compile()/contract() and num_ops(): code that drives a BinaryContraction*
// (EinsumNode, the bench harnesses) works unchanged with BinaryContractionHip.
#ifndef EINSUM_IR_BACKEND_BINARY_CONTRACTION
#define EINSUM_IR_BACKEND_BINARY_CONTRACTION

#include <cstdint>
#include <map>
#include <vector>
#include "../constants.h"
#include "MemoryManager.h"

namespace einsum_ir {
  namespace backend {
    class BinaryContraction;
  }
}

class einsum_ir::backend::BinaryContraction {
  public:
    int64_t m_num_dims_left = 0;
    int64_t m_num_dims_right = 0;
    int64_t m_num_dims_out = 0;

    //! borrowed size maps (inner sizes; outer sizes per tensor for views)
    std::map< int64_t, int64_t > const * m_dim_sizes_inner = nullptr;
    std::map< int64_t, int64_t > const * m_dim_sizes_outer_left = nullptr;
    std::map< int64_t, int64_t > const * m_dim_sizes_outer_right = nullptr;
    std::map< int64_t, int64_t > const * m_dim_sizes_outer_out_aux = nullptr;
    std::map< int64_t, int64_t > const * m_dim_sizes_outer_out = nullptr;

    std::map< int64_t, dim_t > m_dim_types;

    //! borrowed dimension-id arrays
    int64_t const * m_dim_ids_left = nullptr;
    int64_t const * m_dim_ids_right = nullptr;
    int64_t const * m_dim_ids_out = nullptr;
    int64_t const * m_dim_ids_permute_left = nullptr;
    int64_t const * m_dim_ids_permute_right = nullptr;

    std::vector< int64_t > const * m_loop_ids_ext = nullptr;
    std::vector< int64_t > m_loop_ids_int;

    std::vector< dim_t > m_dim_types_out;

    int64_t m_num_dims_c = 0;
    int64_t m_num_dims_m = 0;
    int64_t m_num_dims_n = 0;
    int64_t m_num_dims_k = 0;
    int64_t m_num_dims_i = 0;
    int64_t m_num_dims_j = 0;

    std::vector< int64_t > m_dim_ids_c;
    std::vector< int64_t > m_dim_ids_m;
    std::vector< int64_t > m_dim_ids_n;
    std::vector< int64_t > m_dim_ids_k;
    std::vector< int64_t > m_dim_ids_i;
    std::vector< int64_t > m_dim_ids_j;

    std::vector< int64_t > m_sizes_c;
    std::vector< int64_t > m_sizes_m;
    std::vector< int64_t > m_sizes_n;
    std::vector< int64_t > m_sizes_k;
    std::vector< int64_t > m_sizes_i;
    std::vector< int64_t > m_sizes_j;

    data_t m_dtype_left = UNDEFINED_DTYPE;
    data_t m_dtype_right = UNDEFINED_DTYPE;
    data_t m_dtype_comp = UNDEFINED_DTYPE;
    data_t m_dtype_out = UNDEFINED_DTYPE;

    kernel_t m_ktype_first_touch = UNDEFINED_KTYPE;
    kernel_t m_ktype_main = UNDEFINED_KTYPE;
    kernel_t m_ktype_last_touch = UNDEFINED_KTYPE;

    bool m_compiled = false;

    MemoryManager * m_memory = nullptr;

    int64_t m_num_threads = 1;

    /**
     * Types of the dims of t2 relative to t0 and t1: exclusive to t2, shared
     * with t0 only, with t1 only, or with both.  Repeated ids match distinct
     * occurrences (reference BinaryContraction.cpp:7-60).
     **/
    static void dim_types( int64_t         i_num_dims_t0,
                           int64_t         i_num_dims_t1,
                           int64_t         i_num_dims_t2,
                           int64_t const * i_dim_ids_t0,
                           int64_t const * i_dim_ids_t1,
                           int64_t const * i_dim_ids_t2,
                           dim_t           i_dim_type_t2,
                           dim_t           i_dim_type_t2_t0,
                           dim_t           i_dim_type_t2_t1,
                           dim_t           i_dim_type_t2_t0_t1,
                           dim_t         * o_dim_types_t2 );

    /** Dimension types of left (C/M/K/I), right (C/N/K/J) and out (C/M/N). **/
    static void dim_types( int64_t                      i_num_dims_left,
                           int64_t                      i_num_dims_right,
                           int64_t                      i_num_dims_out,
                           int64_t              const * i_dim_ids_left,
                           int64_t              const * i_dim_ids_right,
                           int64_t              const * i_dim_ids_out,
                           std::vector< dim_t >       * o_dim_types_left,
                           std::vector< dim_t >       * o_dim_types_right,
                           std::vector< dim_t >       * o_dim_types_out );

    /** Ids of the dims of a tensor that have the given type; returns their count. **/
    static int64_t filter_dim_ids( int64_t         i_num_dims_tensor,
                                   dim_t           i_dim_type_filter,
                                   dim_t   const * i_dim_types_tensor,
                                   int64_t const * i_dim_ids_tensor,
                                   int64_t       * o_dim_ids_filtered );

    /** Output dim types and the C/M/N (output order), K/I (left order), J (right order) ids. **/
    static void dim_types_ids( int64_t                        i_num_dims_left,
                               int64_t                        i_num_dims_right,
                               int64_t                        i_num_dims_out,
                               int64_t                const * i_dim_ids_left,
                               int64_t                const * i_dim_ids_right,
                               int64_t                const * i_dim_ids_out,
                               std::vector< dim_t >         * o_dim_types_out,
                               std::vector< int64_t >       * o_dim_ids_c,
                               std::vector< int64_t >       * o_dim_ids_m,
                               std::vector< int64_t >       * o_dim_ids_n,
                               std::vector< int64_t >       * o_dim_ids_k,
                               std::vector< int64_t >       * o_dim_ids_i,
                               std::vector< int64_t >       * o_dim_ids_j );

    /** Row-major element strides keyed by dim id; dims of size < 2 get stride 0. **/
    static void strides( int64_t                              i_num_dims,
                         int64_t                      const * i_dim_ids,
                         std::map< int64_t, int64_t > const * i_dim_sizes,
                         std::map< int64_t, int64_t >       * o_strides );

    virtual ~BinaryContraction() {}

    /** 18-argument init (reference BinaryContraction.h:279-297). **/
    void init( int64_t                              i_num_dims_left,
               int64_t                              i_num_dims_right,
               int64_t                              i_num_dims_out,
               std::map< int64_t, int64_t > const * i_dim_sizes_inner,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_left,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_right,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_out_aux,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_out,
               int64_t                      const * i_dim_ids_left,
               int64_t                      const * i_dim_ids_right,
               int64_t                      const * i_dim_ids_out,
               data_t                               i_dtype_left,
               data_t                               i_dtype_right,
               data_t                               i_dtype_comp,
               data_t                               i_dtype_out,
               kernel_t                             i_ktype_first_touch,
               kernel_t                             i_ktype_main,
               kernel_t                             i_ktype_last_touch,
               int64_t                              i_num_threads );

    /** 23-argument init (reference BinaryContraction.h:326-348). **/
    void init( int64_t                              i_num_dims_left,
               int64_t                              i_num_dims_right,
               int64_t                              i_num_dims_out,
               std::map< int64_t, int64_t > const * i_dim_sizes_inner,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_left,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_right,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_out_aux,
               std::map< int64_t, int64_t > const * i_dim_sizes_outer_out,
               std::vector< int64_t >       const * i_loop_ids_ext,
               int64_t                      const * i_dim_ids_left,
               int64_t                      const * i_dim_ids_right,
               int64_t                      const * i_dim_ids_out,
               int64_t                      const * i_dim_ids_permute_left,
               int64_t                      const * i_dim_ids_permute_right,
               MemoryManager                      * i_memory,
               data_t                               i_dtype_left,
               data_t                               i_dtype_right,
               data_t                               i_dtype_comp,
               data_t                               i_dtype_out,
               kernel_t                             i_ktype_first_touch,
               kernel_t                             i_ktype_main,
               kernel_t                             i_ktype_last_touch,
               int64_t                              i_num_threads );

    /** Derives dim types/ids/sizes (reference BinaryContraction.cpp:352-432). **/
    err_t compile_base();

    virtual err_t compile() = 0;

    virtual void contract( void const * i_tensor_left,
                           void const * i_tensor_right,
                           void       * io_tensor_out ) = 0;

    virtual void contract( void const * i_tensor_left,
                           void const * i_tensor_right,
                           void const * i_tensor_out_aux,
                           void       * io_tensor_out ) = 0;

    /** 2*C*M*N*K, minus C*M*N for a ZERO first touch (reference BinaryContraction.cpp:434-464). **/
    int64_t num_ops();
};

#endif
