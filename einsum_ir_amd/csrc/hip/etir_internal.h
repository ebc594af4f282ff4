// Internal declarations shared by the planner, the kernels and the C ABI of
// libeinsum_ir_hip.so.  Host-only structures; the kernels receive the *Args
// structs by value.
#ifndef ETIR_INTERNAL_H
#define ETIR_INTERNAL_H

#include <cstdint>
#include <memory>
#include <string>
#include <type_traits>
#include <vector>
#include <hip/hip_runtime.h>
#include "../../../include/einsum_ir_hip.h"

namespace etir {

// ---------------------------------------------------------------------------
// error handling
// ---------------------------------------------------------------------------
void set_error( std::string const & msg );
int  fail( int code, std::string const & msg );

#define ETIR_HIP_CHECK( expr )                                                  \
  do {                                                                          \
    hipError_t l_e = ( expr );                                                  \
    if( l_e != hipSuccess ) {                                                   \
      return ::etir::fail( ETIR_UNDEFINED_ERROR,                                \
                           std::string( #expr " failed: " ) +                   \
                           hipGetErrorString( l_e ) );                          \
    }                                                                           \
  } while( 0 )

inline int64_t dtype_bytes( int32_t dt ) {
  if( dt == ETIR_FP32 ) return 4;
  if( dt == ETIR_FP64 ) return 8;
  if( dt == ETIR_BF16 ) return 2;
  return -1;
}

// ---------------------------------------------------------------------------
// permutation
// ---------------------------------------------------------------------------
constexpr int kPermMaxDims = 12;

enum class PermMode : int32_t {
  FILL      = 0,  // ZERO: out = 0 over the output's strides
  TRANSPOSE = 1,  // LDS-tiled 2-D transpose of (in-unit dim, out-unit dim) + batch
  COPY_VEC  = 2,  // both innermost dims unit-stride: vectorised strided copy
  GATHER    = 3,  // anything else: one thread per output element
  TILED     = 4,  // small unit-stride dims: tiles over both tensors' innermost runs
  REG4      = 5,  // short unit-stride dims: 4 x 4 register transposes, 16-byte rows through LDS
  ROWS      = 6   // shared short unit-stride dim: tiles of whole rows, both sides' runs contiguous
};

constexpr int kPermTileDims = 4;   // dims of a TILED tile (2 per run at most)

struct PermArgs {
  void const * in;
  void       * out;
  int32_t  num_batch;                   // number of batch dims (outer -> inner)
  int64_t  batch_size[kPermMaxDims];
  int64_t  batch_s_in[kPermMaxDims];
  int64_t  batch_s_out[kPermMaxDims];
  int64_t  size_i;    // TRANSPOSE: unit-stride dim of the input; COPY_VEC: the common inner dim
  int64_t  size_o;    // TRANSPOSE: unit-stride dim of the output
  int64_t  s_in_o;    // input stride of the o dim
  int64_t  s_out_i;   // output stride of the i dim
  int64_t  tiles_i;
  int64_t  tiles_o;
  int64_t  num_batch_total;
  int64_t  num_elements;
  int32_t  add;       // ktype ADD: out += in
  int32_t  vec_ok;    // 16-byte vector accesses are legal (sizes/strides/alignment)
  // TILED: tile dims (size, extent, strides, tiles along it), tile element
  // count, LDS padding (elements after every 64) and the offset tables, one
  // entry per V consecutive elements: tab_r the input offset of an entry in
  // input order, tab_w {output offset, input-order index of the first
  // element} of an entry in output order (the others tile_t_step apart), and
  // for edge tiles only tab_rc / tab_wc the entries' packed coordinates
  // (8 bits per tile dim)
  int32_t  tile_nd;
  int32_t  tile_n;
  int32_t  tile_pad;
  int32_t  tile_t_step;
  int64_t  tile_size[kPermTileDims];
  int64_t  tile_ext[kPermTileDims];
  int64_t  tile_s_in[kPermTileDims];
  int64_t  tile_s_out[kPermTileDims];
  int64_t  tile_nblk[kPermTileDims];
  int32_t const * tab_r;
  int32_t const * tab_w;
  int32_t const * tab_rc;
  int32_t const * tab_wc;
  // REG4: the dim next to the unit-stride ones in the thread order (size,
  // strides) and how many of its indices one workgroup covers
  int64_t  c_size;
  int64_t  c_s_in;
  int64_t  c_s_out;
  int32_t  c_chunk;
  int64_t  c_nblk;    // workgroups along c (set at launch)
  int32_t  vec_wide;  // COPY_VEC / FILL, bf16: 8-element (16-byte) vectors allowed
  int32_t  slot_pi;   // REG4: LDS pitch (16-byte slots) of i and of c
  int32_t  slot_pc;
  int32_t  nt_store;  // TRANSPOSE: streaming (non-temporal) output stores
  // TRANSPOSE, 2-byte 16-byte-read tile: o1_size > 0 folds the output's
  // next dim (output stride o1_size, input stride s_in_o2) into o, which then
  // runs over o1 + o1_size * o2 (size_o = o1_size * that dim's size);
  // o1_magic = ceil(2^32 / o1_size), so o / o1_size = umulhi(o, o1_magic)
  int32_t  o1_size;
  uint32_t o1_magic;
  int64_t  s_in_o2;
  // ROWS: rows of the shared unit-stride dim (g chunks of the kernel's vector
  // width each); x continues the input's run, y the output's; tiles of
  // rows_ex x rows_ey rows, parked in LDS at rows_pitch chunks per x
  int32_t  rows_g;
  int32_t  rows_ex;
  int32_t  rows_ey;
  int32_t  rows_pitch;
  int64_t  rows_nx;
  int64_t  rows_ny;
  int64_t  rows_nbx;
  int64_t  rows_nby;
  int64_t  rows_s_in_y;
  int64_t  rows_s_out_x;
};

struct PermutePlan {
  PermMode mode = PermMode::GATHER;
  int32_t  reg4_cpt = 1;                 // REG4: passes of the threads over c per workgroup (1, 2 or 4)
  int32_t  reg4_threads = 256;           // REG4: threads per workgroup (64 ... 512)
  bool     reg4_direct = false;          // REG4: rows stored from registers, no LDS exchange
  int32_t  reg4_vb = 4;                  // REG4: block side (bf16: 8 when both unit dims allow)
  int32_t  dtype = ETIR_FP32;
  int32_t  ktype = ETIR_KTYPE_COPY;
  int64_t  elem_bytes = 4;
  int64_t  num_elements = 0;
  int32_t  num_dims = 0;                 // fused dims (output order)
  int64_t  size[kPermMaxDims];
  int64_t  s_in[kPermMaxDims];
  int64_t  s_out[kPermMaxDims];
  PermArgs args{};                       // pointers filled at execute time
  void *   d_tables = nullptr;           // TILED: device offset tables (owned)
  int32_t  tile_vw = 1;                  // TILED: elements per table entry (1 or 4)
  int32_t  rows_vw = 1;                  // ROWS: elements per chunk (16, 8 or 4 bytes; 1 element when unaligned)
  int32_t  tr_shape = 0;                 // TRANSPOSE: tile 64 x 64 (0), 128 x 32 (1) or 32 x 128 (2), i x o;
                                         // 2-byte elements with 16-byte reads: 128 x 64 (3), 128 x 32 (4)
  int64_t  rows_len = 0;                 // ROWS: row length (elements of the shared unit-stride dim)
};

// frees the device memory of a permutation plan
void release_permute( PermutePlan & plan );

int  plan_permute( int64_t         num_dims,
                   int64_t const * sizes,
                   int64_t const * strides_in,
                   int64_t const * strides_out,
                   int32_t         dtype,
                   int32_t         ktype,
                   PermutePlan   & plan );
int  launch_permute( PermutePlan const & plan,
                     void const        * in,
                     void              * out,
                     hipStream_t         stream );

// ---------------------------------------------------------------------------
// contraction
// ---------------------------------------------------------------------------
// Operand load modes of the contraction kernel.  "A" is the operand whose
// dimension indexes the MFMA rows (kernel-M), "B" the MFMA columns (kernel-N).
enum LoadMode : int32_t {
  LOAD_SCALAR  = 0,  // element gathers through the offset tables
  LOAD_VEC_MN  = 1,  // 16-byte vectors along the operand's M (or N) index
  LOAD_VEC_K   = 2,  // 16-byte vectors along K
  LOAD_VEC8_MN = 3,  // 8-byte vectors along M (or N): fp32 runs of even length
  LOAD_VEC8_K  = 4   // 8-byte vectors along K (generic fp32 tiles only)
};

// LDS layout of a load mode: [k][row] for the M/N vector modes, [row][k]
// otherwise
constexpr int32_t lds_layout( int32_t mode ) {
  return ( mode == LOAD_VEC_MN || mode == LOAD_VEC8_MN ) ? LOAD_VEC_MN
       : ( mode == LOAD_VEC8_K ) ? LOAD_VEC_K : mode;
}

// Calls fn( MA, MB, KAFF ) with std::integral_constant arguments equal to the
// run-time operand load modes and affine-K flag, so that a launcher names its
// kernel template once and every mode combination is instantiated from it.
// The 8-byte modes are instantiated only where VEC8 is set.  Unknown modes
// fail with ETIR_COMPILATION_FAILED.
template< bool VEC8 = false, class Fn >
int with_load_modes( int32_t ma, int32_t mb, bool kaff, Fn && fn ) {
  auto pick_k = [&]( auto i_ma, auto i_mb ) -> int {
    if( kaff ) return fn( i_ma, i_mb, std::true_type() );
    return fn( i_ma, i_mb, std::false_type() );
  };
  auto pick_b = [&]( auto i_ma ) -> int {
    switch( mb ) {
      case LOAD_SCALAR: return pick_k( i_ma, std::integral_constant< int32_t, LOAD_SCALAR >() );
      case LOAD_VEC_MN: return pick_k( i_ma, std::integral_constant< int32_t, LOAD_VEC_MN >() );
      case LOAD_VEC_K:  return pick_k( i_ma, std::integral_constant< int32_t, LOAD_VEC_K >() );
      default: break;
    }
    if constexpr( VEC8 ) {
      if( mb == LOAD_VEC8_MN ) return pick_k( i_ma, std::integral_constant< int32_t, LOAD_VEC8_MN >() );
      if( mb == LOAD_VEC8_K )  return pick_k( i_ma, std::integral_constant< int32_t, LOAD_VEC8_K >() );
    }
    return fail( ETIR_COMPILATION_FAILED, "contraction: unknown load mode of operand B" );
  };
  switch( ma ) {
    case LOAD_SCALAR: return pick_b( std::integral_constant< int32_t, LOAD_SCALAR >() );
    case LOAD_VEC_MN: return pick_b( std::integral_constant< int32_t, LOAD_VEC_MN >() );
    case LOAD_VEC_K:  return pick_b( std::integral_constant< int32_t, LOAD_VEC_K >() );
    default: break;
  }
  if constexpr( VEC8 ) {
    if( ma == LOAD_VEC8_MN ) return pick_b( std::integral_constant< int32_t, LOAD_VEC8_MN >() );
    if( ma == LOAD_VEC8_K )  return pick_b( std::integral_constant< int32_t, LOAD_VEC8_K >() );
  }
  return fail( ETIR_COMPILATION_FAILED, "contraction: unknown load mode of operand A" );
}

enum TileCfg : int32_t {
  TILE_F32_128x128 = 0,
  TILE_F32_64x64   = 1,
  TILE_BF16_256x256 = 2,
  TILE_BF16_128x128 = 3,
  TILE_BF16_64x64  = 4,
  TILE_F64_64x64   = 5,
  TILE_BF16_256x128 = 6,
  TILE_BF16_DMA_256x256 = 7,  // direct-to-LDS kernel (contract_dma.h), one workgroup per CU
  TILE_BF16_DMA_256x128 = 8,  // direct-to-LDS kernel, two workgroups per CU
  TILE_CPX_F32_64x64    = 9,  // complex (CPX_MADD) kernels, contract_cpx.hip
  TILE_CPX_F64_64x64    = 10,
  TILE_F32_KWAVE_32x32  = 11, // K split over the waves of one workgroup (contract_kwave.hip)
  TILE_F32_DMA_128x128  = 12, // fp32 direct-to-LDS kernel (contract_f32_dma.hip)
  TILE_GEMV             = 13, // M == 1 or N == 1: one thread per output element (contract_gemv.hip)
  TILE_SKINNY           = 14, // one free side of 2-64: one thread per long index (contract_skinny.hip)
  TILE_PANEL            = 15  // short K, one free side of 65-256 resident in LDS (contract_panel.hip)
};

struct ContractArgs {
  void const * a;
  void const * b;
  void const * aux;
  void       * out;
  // C (batch) offsets per tensor, int64, C entries each
  int64_t const * tc_a;
  int64_t const * tc_b;
  int64_t const * tc_aux;
  int64_t const * tc_out;
  // kernel-M offsets (A, aux, out), kernel-N offsets (B, aux, out), K offsets (A, B)
  int32_t const * tm_a;
  int32_t const * tm_aux;
  int32_t const * tm_out;
  int32_t const * tn_b;
  int32_t const * tn_aux;
  int32_t const * tn_out;
  int32_t const * tk_a;
  int32_t const * tk_b;
  int32_t M, N, K, C;
  int32_t tiles_m, tiles_n;
  // affine K: offset = k * stride (when the K index is one fused dim)
  int32_t k_affine;
  int32_t sk_a, sk_b;
  int32_t first_touch;    // ETIR_KTYPE_{ZERO,COPY,ADD,UNDEFINED}
  int32_t last_touch;     // ETIR_KTYPE_{RELU,ADD,UNDEFINED}
  int32_t k_full;         // K % BK == 0: no K masking needed
  int32_t out_bf16;       // output stored as bf16 (RNE)
  int32_t out_off32;      // every output byte offset (M part + N part, C part excluded) is < 2^32
  int32_t c_inner;        // workgroup ids walk C fastest (the output's unit-stride dim is a C dim)
  int32_t out_nt;         // output columns run in 32-element unit-stride groups: non-temporal stores
  // complex contractions: element offsets of the imaginary parts (A, B, out)
  int64_t cpx_a, cpx_b, cpx_out;
  // affine row tables (tm_a[i] == i * sm_a etc.; -1: not affine), used by
  // kernels that skip the table reads when they can
  int32_t sm_a, sn_b, sm_out, sn_out;
  // persistent direct-to-LDS kernel: start-time stagger, dma_phases groups of
  // workgroups, group p starts p * dma_stagger sleep units (~1 us) late
  int32_t dma_phases, dma_stagger;
  // matrix-vector kernel (kernel M == 1): the long operand B and the output
  // are unit-stride along N with every offset a multiple of 4 elements and
  // N % 4 == 0, so a thread takes 4 consecutive outputs with vector accesses
  int32_t gemv_v4;
  // one-short-side kernel: the long operand is unit-stride along an affine
  // K, every row offset a multiple of 4 elements and K % 4 == 0, so a thread
  // reads its K range in 4-element vectors
  int32_t skinny_kvec;
  // one-short-side kernel: the output is [long][short] with the short side
  // unit-stride, so a workgroup's outputs form one block that it writes in
  // address order through LDS
  int32_t skinny_blk;
  // panel kernel: bytes from the output's base to the end of its last
  // element (stores at or past it are dropped by the buffer range check) and
  // the number of persistent workgroups
  uint32_t out_bytes;
  int32_t  panel_grid;
};

struct ContractionPlan {
  int32_t dtype_in   = ETIR_FP32;
  int32_t dtype_comp = ETIR_FP32;
  int32_t dtype_out  = ETIR_FP32;
  int32_t first_touch = ETIR_KTYPE_UNDEFINED;
  int32_t last_touch  = ETIR_KTYPE_UNDEFINED;
  bool    swapped = false;       // kernel A = right tensor, kernel B = left tensor
  bool    needs_aux = false;
  int64_t C = 1, M = 1, N = 1, K = 1;
  int32_t mode_a = LOAD_SCALAR;
  int32_t mode_b = LOAD_SCALAR;
  int32_t tile = TILE_F32_128x128;
  int32_t tile_fallback = TILE_BF16_256x128;  // used when the DMA kernel's alignment needs fail at launch
  int32_t kwave_waves = 0;                    // TILE_F32_KWAVE_32x32: waves per workgroup and k per wave
  int32_t kwave_kw = 0;
  int32_t dma_variant = 0;                    // 0: BK 64, 2 stages; 1: BK 32, 4 stages, scheduled (VEC_MN x VEC_MN);
                                              // 3: its persistent variant where eligible (else 1)
  int64_t flops = 0;
  int64_t bytes = 0;
  // fused loops per kernel role (outer -> inner) for diagnostics
  std::string desc;
  // device blob with all tables
  void *  d_tables = nullptr;
  ContractArgs args{};          // table pointers + sizes; tensor pointers set at execute
  // split K: the contraction runs as `partial` -- the split K loops turned
  // into C loops that write one slice each of the workspace (laid out like
  // the output, `out_span` elements apart: the output's extent rounded up to
  // 64) -- followed by split_reduce, which sums the slices in a fixed order
  // and applies the touch kernels.  out_dense: the output's C, M and N
  // offsets are exactly 0 .. out_dense - 1 (a dense tensor), so the
  // reduction runs over that range as flat arrays (0: not dense)
  int32_t split = 1;
  int64_t out_span = 0;
  int64_t out_dense = 0;
  // out_dense with an aux tensor: the aux offset of output offset o is
  // o % out_dense_aux (the aux broadcasts over the output's outermost loops
  // and matches its strides on the others)
  int64_t out_dense_aux = 0;
  void *  d_ws = nullptr;
  std::shared_ptr< ContractionPlan > partial;
  // tables and workspace live in a caller's region (DevicePlacement), not in
  // memory the plan allocated and frees
  bool    placed = false;
};

// Where a plan's device memory comes from when it may not allocate: a
// region the caller provides (the scratch array of the allocation-free entry
// point), handed out front to back in 256-byte aligned pieces.  The offset
// tables are then written by a kernel on `stream` from the loop sizes and
// strides (no host-to-device copy).
struct DevicePlacement {
  char *      base     = nullptr;
  std::size_t capacity = 0;
  std::size_t used     = 0;
  hipStream_t stream   = nullptr;
};

// One group of offset tables over the same loops (outer -> inner): entry e
// of table t is sum_d digit_d(e) * strides[t][d], the mixed-radix digits of e
// with the innermost loop fastest.  Written as int64 (is64) or int32 at byte
// offset dst[t] from the region's base.
constexpr int kFillMaxDims = 16;
struct TableFill {
  int64_t count;
  int64_t dst[4];
  int64_t sizes[kFillMaxDims];
  int64_t strides[4][kFillMaxDims];
  int32_t ndims;
  int32_t ntab;
  int32_t is64;
};
int launch_fill_tables( TableFill const & f, char * base, hipStream_t stream );

// frees the device memory of a contraction plan (tables, workspace, partial plan)
void release_contraction( ContractionPlan & plan );

struct SplitReduceArgs {
  float const * ws;
  void const  * aux;
  void        * out;
  int64_t const * tc_out;
  int64_t const * tc_aux;
  int32_t const * tm_out;
  int32_t const * tm_aux;
  int32_t const * tn_out;
  int32_t const * tn_aux;
  int64_t span;
  int64_t n_flat;     // > 0: out[o] = touch( sum_s ws[s * span + o] ) for o < n_flat, no tables
  int64_t flat_aux;   // n_flat > 0 with an aux tensor: its offset for output offset o is o % flat_aux
  int32_t flat_vec;   // n_flat > 0: 4 elements per thread (span % 4 == 0, output aligned to 4 elements)
  int32_t C, M, N, S;
  int32_t first_touch;
  int32_t last_touch;
  int32_t out_bf16;
};

int launch_split_reduce( SplitReduceArgs const & a, hipStream_t stream );

int  plan_contraction( int64_t            num_loops,
                       int32_t const    * dim_types,
                       int64_t const    * sizes,
                       int64_t const    * strides_left,
                       int64_t const    * strides_right,
                       int64_t const    * strides_out_aux,
                       int64_t const    * strides_out,
                       int32_t            dtype_left,
                       int32_t            dtype_right,
                       int32_t            dtype_comp,
                       int32_t            dtype_out,
                       int32_t            ktype_first_touch,
                       int32_t            ktype_main,
                       int32_t            ktype_last_touch,
                       ContractionPlan  & plan,
                       DevicePlacement  * place = nullptr );
int  launch_contraction( ContractionPlan const & plan,
                         void const            * left,
                         void const            * right,
                         void const            * out_aux,
                         void                  * out,
                         hipStream_t             stream );

}  // namespace etir

struct etir_plan_s {
  int32_t kind = 0;              // 1 contraction, 2 permutation
  int32_t device = 0;
  etir::ContractionPlan cont;
  etir::PermutePlan     perm;
};

#endif
