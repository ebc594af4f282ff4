// Dimension-ordering primitives of the tree path (drop-in for the parts of
// reference src/backend/BinaryPrimitives.h that EinsumNode uses):
//   swap_inputs  -- which child becomes the left operand
//                   (reference src/backend/BinaryPrimitives.cpp:87-134);
//   init         -- block-size targets per dtype/backend (:25-85; HIP added);
//   reorder      -- internal dimension order of both children for a tensor
//                   ordering (:833-1711) or a backend (:1713-1768);
//   reorder_gpu  -- the HIP backend's own child layouts (no counterpart);
//   blocking     -- the blocked C/M/N/K dims a primitive can take directly
//                   from the tensors' innermost dims (:136-831).
// compileLoopOrder / splitDimension of the reference (:1770-...) are neither
// called by the reference nor covered by its tests and are not provided.
#ifndef EINSUM_IR_BACKEND_BINARY_PRIMITIVES
#define EINSUM_IR_BACKEND_BINARY_PRIMITIVES

#include <cstdint>
#include <map>
#include <vector>
#include "../constants.h"

namespace einsum_ir {
  namespace backend {
    class BinaryPrimitives;
  }
}

class einsum_ir::backend::BinaryPrimitives {
  public:
    int64_t m_size_cb_min = 0;
    int64_t m_size_cb_max = 0;
    int64_t m_size_mb_min = 0;
    int64_t m_size_mb_max = 0;
    int64_t m_size_nb_min = 0;
    int64_t m_size_nb_max = 0;
    int64_t m_size_kb_min = 0;
    int64_t m_size_kb_max = 0;

    //! placement of the blocked C dims inside the inputs
    enum class CBlock { NONE, INNER, OUTER };

    /**
     * Generic reorder used by the three tensor orderings: classifies the
     * trailing output dims into blocked C (per `i_cblock`), blocked M and
     * blocked N groups (size targets min/max), blocks the largest K dims,
     * and writes the new dim orders of the left/right inputs; the output
     * keeps its order.
     **/
    static err_t reorder_generic( CBlock                               i_cblock,
                                  int64_t                              i_size_cb_min,
                                  int64_t                              i_size_cb_max,
                                  int64_t                              i_size_mb_min,
                                  int64_t                              i_size_mb_max,
                                  int64_t                              i_size_nb_min,
                                  int64_t                              i_size_nb_max,
                                  int64_t                              i_size_kb_min,
                                  int64_t                              i_size_kb_max,
                                  int64_t                              i_num_dims_left,
                                  int64_t                              i_num_dims_right,
                                  int64_t                              i_num_dims_out,
                                  std::map< int64_t, int64_t > const * i_dim_sizes,
                                  int64_t                            * io_dim_ids_left,
                                  int64_t                            * io_dim_ids_right,
                                  int64_t                            * io_dim_ids_out );

    void init( int64_t i_size_cb_min, int64_t i_size_cb_max,
               int64_t i_size_mb_min, int64_t i_size_mb_max,
               int64_t i_size_nb_min, int64_t i_size_nb_max,
               int64_t i_size_kb_min, int64_t i_size_kb_max );

    err_t init( data_t    i_data_type,
                backend_t i_backend_type );

    /** True if the inputs have to be swapped so that the output's fastest non-C dim is M. **/
    static bool swap_inputs( int64_t         i_num_dims_left,
                             int64_t         i_num_dims_right,
                             int64_t         i_num_dims_out,
                             int64_t const * i_dim_ids_left,
                             int64_t const * i_dim_ids_right,
                             int64_t const * i_dim_ids_out );

    err_t reorder( tenord_t                             i_primitive_ordering,
                   int64_t                              i_num_dims_left,
                   int64_t                              i_num_dims_right,
                   int64_t                              i_num_dims_out,
                   std::map< int64_t, int64_t > const * i_dim_sizes,
                   int64_t                            * io_dim_ids_left,
                   int64_t                            * io_dim_ids_right,
                   int64_t                            * io_dim_ids_out ) const;

    /**
     * Blocked dims for a primitive blocking (reference BinaryPrimitives.cpp:728-831):
     * walks the tensors from their innermost dims and collects, per type, the
     * dims that are stored contiguously in every tensor that holds them and
     * that keep the block within the size targets of init.  Strides default
     * to the row-major strides of the dim orders when a map is null.
     * Outputs are in row-major order (outermost first).
     **/
    err_t blocking( primblo_t                            i_primitive_blocking,
                    int64_t                              i_num_dims_left,
                    int64_t                              i_num_dims_right,
                    int64_t                              i_num_dims_out,
                    int64_t                      const * i_dim_ids_left,
                    int64_t                      const * i_dim_ids_right,
                    int64_t                      const * i_dim_ids_out,
                    std::map< int64_t, int64_t > const * i_dim_sizes,
                    std::map< int64_t, int64_t > const * i_strides_left,
                    std::map< int64_t, int64_t > const * i_strides_right,
                    std::map< int64_t, int64_t > const * i_strides_out,
                    std::vector< int64_t >             * o_dim_ids_cb,
                    std::vector< int64_t >             * o_dim_ids_mb,
                    std::vector< int64_t >             * o_dim_ids_nb,
                    std::vector< int64_t >             * o_dim_ids_kb ) const;

    /**
     * Internal dim orders of both children for the HIP backend.  No
     * counterpart in the reference: its TPP ordering serves libxsmm's
     * column-major (packed) GEMMs and places the shared C dims innermost,
     * where the GPU kernel -- which runs C loops in its grid and loads
     * 16-byte vectors along an operand's unit-stride M/N or K loop -- has to
     * gather single elements.
     *   - A child the tree computes (i_fixed_* false) is laid out for the
     *     kernel's fastest operand pairing: the operand on the kernel's row
     *     side M/N-contiguous ([C, I/J, K, own M/N]), the one on the column
     *     side -- the side of the output's unit-stride dim -- K-contiguous
     *     ([C, own M/N, I/J, K]), unless the extents rule out 16-byte vectors
     *     that way.  C and M/N dims follow the output's order, K dims one
     *     order shared by both children, so that they fuse.
     *   - A child whose layout is given (i_fixed_* true: a leaf) keeps it when
     *     the kernel reads it with vector loads as it is -- innermost dim a K
     *     dim, or an M/N dim on the row side (the output's innermost row-side
     *     dim when the output's unit-stride run is shorter than 32 elements,
     *     so that neighbouring tile rows are neighbours in memory), or the
     *     output's innermost dim on the column side, with a size that is a
     *     multiple of the vector width
     *     i_vec -- or when the element gathers it needs (its bytes times the
     *     tiles of the other side) stay below i_min_bytes_permute; otherwise
     *     it is laid out like a computed child (one permutation of the leaf
     *     per evaluation, none once locked).  Two given children whose
     *     innermost K dims differ cannot both be read along K: the smaller one
     *     is laid out again.
     * The output keeps its order.
     **/
    static err_t reorder_gpu( bool                                 i_fixed_left,
                              bool                                 i_fixed_right,
                              int64_t                              i_vec,
                              int64_t                              i_bytes_per_element,
                              int64_t                              i_min_bytes_permute,
                              int64_t                              i_num_dims_left,
                              int64_t                              i_num_dims_right,
                              int64_t                              i_num_dims_out,
                              std::map< int64_t, int64_t > const * i_dim_sizes,
                              int64_t                            * io_dim_ids_left,
                              int64_t                            * io_dim_ids_right,
                              int64_t                            * io_dim_ids_out );

    err_t reorder( backend_t                            i_backend_type,
                   int64_t                              i_num_dims_left,
                   int64_t                              i_num_dims_right,
                   int64_t                              i_num_dims_out,
                   std::map< int64_t, int64_t > const * i_dim_sizes,
                   int64_t                            * io_dim_ids_left,
                   int64_t                            * io_dim_ids_right,
                   int64_t                            * io_dim_ids_out ) const;
};

#endif
