// gfx950 bf16 contraction kernel with direct-to-LDS operand loads.
//
// Same contraction and epilogue as contract_kernel.h
//   out[c][m][n] = touch( sum_k A[c][m][k] * B[c][n][k] )
// (first/last-touch semantics of reference src/basic/binary/
// ContractionBackendTpp.cpp:15-49,127-163, applied once per output element),
// specialised for the large, compute-bound case:
//
// * bf16 operands, fp32 accumulation, v_mfma_f32_32x32x16_bf16;
// * one workgroup of 4 waves per CU computes a BM x BN = 256 x 256 tile, each
//   wave a 128 x 128 block (16 accumulator tiles of 32 x 32 = 256 registers),
//   which keeps the LDS read traffic at (128 + 128) rows per wave and k;
// * operands go global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
//   staging, no ds_write): one instruction moves 64 x 16 bytes into one
//   contiguous KiB of LDS, lane i into bytes [16 i, 16 i + 16).  Each lane
//   chooses WHICH 16 global bytes it fetches, which is how the XOR swizzle
//   below is applied.  Out-of-range rows and k read as zero through the
//   buffer's range check (offset >= num_records), so edge tiles need no
//   branches;
// * STAGES LDS buffers: the loads for k-step t + STAGES - 1 are issued at the
//   start of step t, so a load has STAGES - 1 steps of MFMA work to land.
//
// Operand layouts in LDS (per stage), both read with conflict-free patterns:
//
// VEC_MN (16-byte runs along the operand's rows, e.g. M-contiguous A):
//   [k][R] bf16, R*2 bytes per k row, 16-byte segment g of k row k stored at
//   segment g ^ swz(k & 3), swz = {0, 6, 10, 12}.  MFMA fragments are read with
//   ds_read_b64_tr_b16 (the LDS transpose read of gfx950); one such read
//   touches 4 k rows x 64 bytes, which the swizzle spreads over disjoint bank
//   ranges for 16-lane (128 B/clk) and 32-lane (256 B/clk) service groups.
// VEC_K (16-byte runs along K, K-contiguous operand):
//   [R][BK] bf16, segment g (8 k) of row r stored at g ^ swz(r),
//   swz(r) = (r & 7) ^ ((r >> 3) & 1); fragments are ds_read_b128.
#ifndef ETIR_CONTRACT_DMA_H
#define ETIR_CONTRACT_DMA_H

#include "contract_kernel.h"

namespace etir {
namespace kern {

typedef int32_t i32x4 __attribute__( ( ext_vector_type( 4 ) ) );

// buffer resource of a raw (stride 0) buffer: base address, num_records
// bytes, gfx9 word-3 format bits for untyped dword access
__device__ inline i32x4 make_rsrc( void const * base, uint32_t num_records ) {
  uint64_t const l_b = reinterpret_cast< uint64_t >( uniform_ptr( base ) );
  i32x4 l_r;
  l_r[0] = int32_t( uint32_t( l_b ) );
  l_r[1] = int32_t( uint32_t( l_b >> 32 ) & 0xffffu );
  l_r[2] = int32_t( num_records );
  l_r[3] = 0x00020000;
  return l_r;
}

// 64 lanes x 16 bytes global -> LDS: lane i's bytes at buffer offset voff go
// to LDS byte lds_addr + 16 i.  Written as inline assembly so that the
// compiler neither tracks these loads (it would otherwise wait for all of
// them before any LDS read, which defeats the prefetch) nor moves them across
// the explicit waits and barriers of the main loop; M0 carries the LDS base
// and is not used by anything else in these kernels.  gfx9 needs one wait
// state between an SALU write of M0 and an LDS-DMA instruction reading it
// (the compiler's hazard recognizer does not look inside inline assembly).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void dma16( i32x4 rsrc, uint32_t voff, uint32_t lds_addr ) {
  asm volatile( "s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                :: "v"( voff ), "s"( rsrc ), "s"( lds_addr ) : "m0" );
}
#pragma clang diagnostic pop

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// The same load with the lane's row offset in voff and a wave-uniform byte
// offset (the k step) in soff: global address base + voff + soff, LDS
// address M0 + 16 i.  M0 must have been written beforehand (set_m0*);
// INC > 0 advances M0 by INC after the load, for the next chunk (the
// instructions between two issues cover the wait state an LDS-DMA
// instruction needs after an SALU write of M0).  No instruction offset: it
// would move the global and the LDS address alike.
template< int INC >
__device__ inline void dma16_so( i32x4 rsrc, uint32_t voff, uint32_t soff ) {
  if constexpr( INC > 0 ) {
    asm volatile( "buffer_load_dwordx4 %0, %1, %2 offen lds\n\ts_add_u32 m0, %3, m0"
                  :: "v"( voff ), "s"( rsrc ), "s"( soff ), "n"( INC ) : "m0", "scc" );
  }
  else {
    asm volatile( "buffer_load_dwordx4 %0, %1, %2 offen lds" :: "v"( voff ), "s"( rsrc ), "s"( soff ) );
  }
}

// M0 = v (with the wait state an LDS-DMA instruction needs after an SALU
// write of M0)
__device__ inline void set_m0( uint32_t v ) {
  asm volatile( "s_mov_b32 m0, %0\n\ts_nop 0" :: "s"( v ) : "m0" );
}

// M0 = base + IMM
template< uint32_t IMM >
__device__ inline void set_m0_add( uint32_t base ) {
  asm volatile( "s_add_u32 m0, %0, %1\n\ts_nop 0" :: "s"( base ), "n"( IMM ) : "m0", "scc" );
}
#pragma clang diagnostic pop

// LDS byte address of a generic pointer into a __shared__ array
__device__ inline uint32_t lds_addr( void const * p ) {
  return uint32_t( reinterpret_cast< uintptr_t >( (__attribute__( ( address_space( 3 ) ) ) char const *) p ) );
}

// wait until at most N vector-memory operations of this wave are in flight
template< int N >
__device__ inline void wait_vmcnt() {
  static_assert( N >= 0 && N < 64, "vmcnt out of range" );
  asm volatile( "s_waitcnt vmcnt(%0)" :: "n"( N ) : "memory" );
}

// workgroup barrier that also orders LDS accesses around it (no waitcnt)
__device__ inline void barrier_lds() {
  asm volatile( "s_barrier" ::: "memory" );
}

__device__ inline void wait_lgkmcnt0() {
  asm volatile( "s_waitcnt lgkmcnt(0)" ::: "memory" );
}

// byte offset used for lanes whose row or k is out of range: at or above the
// buffer's num_records, so the load returns zeros
constexpr uint32_t kDmaOob = 0x80000000u;

__device__ inline uint32_t swz_mn( int k ) {
  return ( 0xCA60u >> ( 4 * ( k & 3 ) ) ) & 0xFu;
}

__device__ inline uint32_t swz_k( int r ) {
  return uint32_t( ( r & 7 ) ^ ( ( r >> 3 ) & 1 ) );
}

// ---------------------------------------------------------------------------
// DMA loaders: precomputed per-lane byte offsets (row part + local k part);
// the k-step part is added per issue.
// ---------------------------------------------------------------------------
template< int R, int BK, int W, int MODE >
struct DmaLoader;

template< int R, int BK, int W >
struct DmaLoader< R, BK, W, LOAD_VEC_MN > {
  static constexpr int SEGS  = R / 8;          // 16-byte segments per k row
  static constexpr int KPC   = 64 / SEGS;      // k rows per KiB chunk
  static constexpr int NCH   = BK / KPC;       // chunks per stage
  static constexpr int NJ    = NCH / W;        // chunks per wave
  static constexpr int STAGE_BYTES = BK * R * 2;
  static_assert( SEGS >= 16 && SEGS <= 64 && 64 % SEGS == 0, "VEC_MN DMA: R must be 128..512" );
  static_assert( NCH % W == 0, "VEC_MN DMA: chunks must divide over the waves" );

  uint32_t m_off[NJ];
  int32_t  m_kk[NJ];
  uint32_t m_valid;    // bit j: chunk j's row is inside the operand

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0, int32_t sk,
                               int wave, int lane ) {
    load_rows( tab_rows, rows, row0, wave, lane );
    finalize( sk );
  }

  // first half of init: reads the row offsets (clamped index, unconditional)
  // into m_off without using them, so the loads can be issued long before
  // finalize() without forcing a wait
  __device__ inline void load_rows( int32_t const * tab_rows, int32_t rows, int32_t row0, int wave, int lane ) {
    m_valid = 0;
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      int const l_chunk = wave * NJ + l_j;
      int const l_kk = l_chunk * KPC + lane / SEGS;
      int const l_p  = lane % SEGS;
      int const l_g  = l_p ^ int( swz_mn( l_kk ) );
      int32_t const l_row = row0 + 8 * l_g;
      m_kk[l_j] = l_kk;
      if( l_row < rows ) m_valid |= 1u << l_j;
      m_off[l_j] = uint32_t( tab_rows[min( l_row, rows - 1 )] );
    }
  }

  // second half: byte offsets of the lane's 16-byte segment in k-step 0
  __device__ inline void finalize( int32_t sk ) {
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      m_off[l_j] = ( ( m_valid >> l_j ) & 1u ) ? uint32_t( 2 * ( int32_t( m_off[l_j] ) + m_kk[l_j] * sk ) ) : kDmaOob;
    }
  }

  // k0: first k of the step; kstep_bytes = 2 * k0 * sk.  Lanes whose k is at
  // or past K (partial last step, prefetches beyond the last step) load zeros.
  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline void issue_one( i32x4 rsrc, uint32_t lds_stage, int wave,
                                                                       int32_t k0, int32_t K,
                                                                       uint32_t kstep_bytes ) {
    uint32_t l_off = m_off[J] + kstep_bytes;
    if( k0 + m_kk[J] >= K ) l_off = kDmaOob;
    dma16( rsrc, l_off, lds_stage + ( wave * NJ + J ) * 1024 );
  }
  // chunk J with M0 at this wave's chunk J of the stage (set_m0 before
  // chunk 0, advanced by each issue) and the k step's bytes in soffset
  template< int J, bool CHK >
  __device__ __attribute__( ( always_inline ) ) inline void issue_so( i32x4 rsrc, uint32_t kstep_bytes, int32_t k0,
                                                                      int32_t K ) {
    uint32_t l_off = m_off[J];
    if( CHK && k0 + m_kk[J] >= K ) l_off = kDmaOob;
    dma16_so< ( J + 1 < NJ ) ? 1024 : 0 >( rsrc, l_off, kstep_bytes );
  }
  __device__ inline void issue( i32x4 rsrc, uint32_t lds_stage, int wave, int32_t k0,
                                int32_t K, uint32_t kstep_bytes ) {
    static_for< NJ >( [&]( auto jc ) __attribute__( ( always_inline ) ) {
      issue_one< decltype( jc )::value >( rsrc, lds_stage, wave, k0, K, kstep_bytes );
    } );
  }
};

template< int R, int BK, int W >
struct DmaLoader< R, BK, W, LOAD_VEC_K > {
  static constexpr int SEGS  = BK / 8;         // 16-byte segments per row
  static constexpr int RPC   = 64 / SEGS;      // rows per KiB chunk
  static constexpr int NCH   = R / RPC;
  static constexpr int NJ    = NCH / W;
  static constexpr int STAGE_BYTES = BK * R * 2;
  static_assert( SEGS == 8, "VEC_K DMA: BK must be 64" );
  static_assert( NCH % W == 0, "VEC_K DMA: chunks must divide over the waves" );

  uint32_t m_off[NJ];
  int32_t  m_kl[NJ];   // local k of this lane's segment in chunk j

  __device__ inline void init( int32_t const * tab_rows, int32_t rows, int32_t row0, int32_t sk,
                               int wave, int lane ) {
    int const l_p = lane % SEGS;
#pragma unroll
    for( int l_j = 0; l_j < NJ; l_j++ ) {
      int const l_r   = ( wave * NJ + l_j ) * RPC + lane / SEGS;
      int const l_g   = l_p ^ int( swz_k( l_r ) );
      int32_t const l_row = row0 + l_r;
      m_off[l_j] = ( l_row < rows ) ? uint32_t( 2 * ( tab_rows[l_row] + 8 * l_g * sk ) ) : kDmaOob;
      m_kl[l_j]  = 8 * l_g;
    }
  }

  template< int J >
  __device__ __attribute__( ( always_inline ) ) inline void issue_one( i32x4 rsrc, uint32_t lds_stage, int wave,
                                                                       int32_t k0, int32_t K,
                                                                       uint32_t kstep_bytes ) {
    uint32_t const l_off = ( k0 + m_kl[J] < K ) ? m_off[J] + kstep_bytes : kDmaOob;
    dma16( rsrc, l_off, lds_stage + ( wave * NJ + J ) * 1024 );
  }
  __device__ inline void issue( i32x4 rsrc, uint32_t lds_stage, int wave, int32_t k0,
                                int32_t K, uint32_t kstep_bytes ) {
    static_for< NJ >( [&]( auto jc ) __attribute__( ( always_inline ) ) {
      issue_one< decltype( jc )::value >( rsrc, lds_stage, wave, k0, K, kstep_bytes );
    } );
  }
};

// ---------------------------------------------------------------------------
// fragment readers: per-lane byte addresses for each 32-row block, k-substep
// offsets are immediates
// ---------------------------------------------------------------------------
template< int R, int BK, int NB, int MODE >
struct DmaFrag;

template< int R, int BK, int NB >
struct DmaFrag< R, BK, NB, LOAD_VEC_MN > {
  typedef short v4i16 __attribute__( ( ext_vector_type( 4 ) ) );
  typedef short v8i16 __attribute__( ( ext_vector_type( 8 ) ) );
  typedef __attribute__( ( address_space( 3 ) ) ) v4i16 lds_v4i16;
  uint32_t m_addr[NB];

  // row0: first row of this wave's NB blocks of 32 rows
  __device__ inline void init( int row0, int lane ) {
    int const l_q  = lane >> 4;
    int const l_L  = lane & 15;
    int const l_kb = 8 * ( l_q >> 1 ) + ( l_L >> 2 );
#pragma unroll
    for( int l_i = 0; l_i < NB; l_i++ ) {
      int const l_row = row0 + 32 * l_i + 16 * ( l_q & 1 ) + 4 * ( l_L & 3 );
      m_addr[l_i] = uint32_t( l_kb * R * 2 ) + ( uint32_t( ( l_row >> 3 ) ^ int( swz_mn( l_kb ) ) ) << 4 )
                  + uint32_t( ( l_row & 7 ) * 2 );
    }
  }

  // fragment (8 consecutive k of one row per lane) of block i, k substep s
  __device__ inline bf16x8 read( char const * lds_stage, int i, int s ) const {
    char const * l_p0 = lds_stage + m_addr[i] + s * 16 * R * 2;
    v4i16 l_lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16( (lds_v4i16 *) ( l_p0 ) );
    v4i16 l_hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16( (lds_v4i16 *) ( l_p0 + 4 * R * 2 ) );
    v8i16 l_all = __builtin_shufflevector( l_lo, l_hi, 0, 1, 2, 3, 4, 5, 6, 7 );
    return __builtin_bit_cast( bf16x8, l_all );
  }

  // the same fragment as two separately issued reads (units 0 and 1)
  static constexpr int UNITS = 2;
  struct Part { v4i16 h[2]; };
  template< int U >
  __device__ __attribute__( ( always_inline ) ) inline void read_unit( char const * lds_stage, int i, int s,
                                                                       Part & f ) const {
    char const * l_p = lds_stage + m_addr[i] + s * 16 * R * 2 + U * 4 * R * 2;
    f.h[U] = __builtin_amdgcn_ds_read_tr16_b64_v4i16( (lds_v4i16 *) l_p );
  }
  __device__ static __attribute__( ( always_inline ) ) inline bf16x8 value( Part const & f ) {
    return __builtin_bit_cast( bf16x8, __builtin_shufflevector( f.h[0], f.h[1], 0, 1, 2, 3, 4, 5, 6, 7 ) );
  }

  // the same addresses + 64 KiB, for reads whose immediate offset would not
  // fit the 16-bit field (made opaque so the compiler keeps them in registers
  // instead of adding 64 KiB before every such read)
  uint32_t m_addr_hi[NB];
  __device__ inline void init_hi() {
#pragma unroll
    for( int l_i = 0; l_i < NB; l_i++ ) {
      asm volatile( "v_add_u32 %0, 0x10000, %1" : "=v"( m_addr_hi[l_i] ) : "v"( m_addr[l_i] ) );
    }
  }
  // unit U of the fragment of block i at compile-time byte offset OFF from
  // the start of LDS (stage, operand and substep offsets folded into OFF)
  template< int U, int OFF >
  __device__ __attribute__( ( always_inline ) ) inline void read_unit_c( char const * lds, int i, Part & f ) const {
    constexpr int l_off = OFF + U * 4 * R * 2;
    static_assert( l_off < 2 * 65536, "LDS offset" );
    uint32_t const l_a = ( l_off >= 65536 ) ? m_addr_hi[i] + uint32_t( l_off - 65536 ) : m_addr[i] + uint32_t( l_off );
    f.h[U] = __builtin_amdgcn_ds_read_tr16_b64_v4i16( (lds_v4i16 *) ( lds + l_a ) );
  }

};

template< int R, int BK, int NB >
struct DmaFrag< R, BK, NB, LOAD_VEC_K > {
  // [R][64] bf16, 128 bytes per row; lane: row = lane % 32, segment 2 s + lane / 32
  uint32_t m_row_addr;
  uint32_t m_seg[BK / 16];

  __device__ inline void init( int row0, int lane ) {
    int const l_r = row0 + ( lane & 31 );
    m_row_addr = uint32_t( l_r * BK * 2 );
#pragma unroll
    for( int l_s = 0; l_s < BK / 16; l_s++ ) {
      m_seg[l_s] = uint32_t( ( 2 * l_s + ( lane >> 5 ) ) ^ int( swz_k( l_r ) ) ) << 4;
    }
  }

  __device__ inline bf16x8 read( char const * lds_stage, int i, int s ) const {
    return *reinterpret_cast< bf16x8 const * >( lds_stage + m_row_addr + m_seg[s] + i * 32 * BK * 2 );
  }

  static constexpr int UNITS = 1;
  struct Part { bf16x8 v; };
  template< int U >
  __device__ __attribute__( ( always_inline ) ) inline void read_unit( char const * lds_stage, int i, int s,
                                                                       Part & f ) const {
    f.v = read( lds_stage, i, s );
  }
  __device__ static __attribute__( ( always_inline ) ) inline bf16x8 value( Part const & f ) { return f.v; }
};

// ---------------------------------------------------------------------------
// compile-time schedule of one k substep (TM x TN MFMAs)
//   reads: A0 (all units), B0, A1, B1, ...
//   MFMAs: (i, j) ordered by the read position of their later operand, so
//          each MFMA of the next substep finds its fragments long landed
// ---------------------------------------------------------------------------
template< int TM, int TN >
struct MfmaOrder {
  int i[TM * TN];
  int j[TM * TN];
  constexpr MfmaOrder() : i(), j() {
    int l_p = 0;
    int const l_kmax = 2 * ( TM > TN ? TM : TN );
    for( int l_key = 0; l_key <= l_kmax; l_key++ )
      for( int l_i = 0; l_i < TM; l_i++ )
        for( int l_j = 0; l_j < TN; l_j++ ) {
          int const l_k = ( 2 * l_i > 2 * l_j + 1 ) ? 2 * l_i : 2 * l_j + 1;
          if( l_k == l_key ) { i[l_p] = l_i; j[l_p] = l_j; l_p++; }
        }
  }
};

// slot (MFMA index) of DMA issue d when ND issues spread over NQ MFMAs
template< int NQ, int ND >
constexpr int dma_slot( int d ) {
  return ( ( d + 1 ) * NQ ) / ND - 1;
}

// number of DMA issues placed before the instruction that follows MFMA q
template< int NQ, int ND >
constexpr int dma_before( int q ) {
  int l_n = 0;
  for( int l_d = 0; l_d < ND; l_d++ ) if( dma_slot< NQ, ND >( l_d ) < q ) l_n++;
  return l_n;
}

template< int TM, int TN, int UA, int UB >
struct ReadOrder {
  static constexpr int U = TM * UA + TN * UB;
  int isb[U];
  int idx[U];
  int unit[U];
  constexpr ReadOrder() : isb(), idx(), unit() {
    int l_r = 0;
    for( int l_f = 0; l_f < ( TM > TN ? TM : TN ); l_f++ ) {
      if( l_f < TM ) for( int l_u = 0; l_u < UA; l_u++ ) { isb[l_r] = 0; idx[l_r] = l_f; unit[l_r] = l_u; l_r++; }
      if( l_f < TN ) for( int l_u = 0; l_u < UB; l_u++ ) { isb[l_r] = 1; idx[l_r] = l_f; unit[l_r] = l_u; l_r++; }
    }
  }
};

// ---------------------------------------------------------------------------
// Main loop with an explicit instruction schedule (BK 32 = two k substeps,
// four LDS stages).  With one wave per SIMD the matrix core idles whenever
// the wave stalls, so every MFMA is followed by the LDS reads of the next
// substep's fragments, the eight DMA issues of a step are spread over all
// of its MFMAs (one per four), and the wait + barrier that publish the next
// stage sit after four MFMAs of the last substep, when the data has long
// landed.  sched_barrier(0) keeps the compiler from regrouping the sequence.
//
// Step t (stage buffer t % 4):
//   substep 0: 16 MFMAs on fragment set 0, reads of substep 1 into set 1
//   substep 1: 4 MFMAs on set 1; wait for step t + 1 (own DMA: vmcnt,
//              everyone's: barrier); 12 MFMAs with the reads of step t + 1,
//              substep 0 into set 0
//   throughout: DMA of step t + 3 into the buffer of step t - 1 (freed by
//              the barrier that ended step t - 1)
// The last three steps issue no DMA (vmcnt(0) before the barrier) and the
// final step has no barrier.
//
// Issue cost: with one wave per SIMD every instruction between two MFMAs
// delays the next one, so the steady loop carries as few as it can (about
// 100 per step of 32 MFMAs, from about 150): the steps whose loads are whole
// k steps skip the per-lane K test; a DMA issue takes the k step's bytes in
// soffset (no per-lane add) and M0 is written once per operand and step, then
// advanced by 1 KiB after each issue; and the loop runs in groups of STAGES
// steps whose stage index is a compile-time constant, so every fragment
// read's LDS address is a base register plus an immediate (config 3:
// 259.5 -> 244.5 us per launch, the K test alone 10 us of it).
// ---------------------------------------------------------------------------
// prologue of the main loop: the loads of k-steps 0 .. STAGES-2 (steps >= nk
// load zeros) into stage buffers 0 .. STAGES-2
template< int BK, int STAGES, typename LdA, typename LdB >
__device__ __attribute__( ( always_inline ) ) inline void prologue_issue( char * l_lds, LdA & l_lda, LdB & l_ldb,
                                                                          i32x4 l_ra, i32x4 l_rb, int l_wave,
                                                                          int32_t l_K, uint32_t l_kb_a,
                                                                          uint32_t l_kb_b ) {
  constexpr int SA = LdA::STAGE_BYTES;
  constexpr int SB = LdB::STAGE_BYTES;
  uint32_t const l_lds0 = lds_addr( l_lds );
#pragma unroll
  for( int l_t = 0; l_t < STAGES - 1; l_t++ ) {
    uint32_t const l_st = l_lds0 + uint32_t( l_t ) * ( SA + SB );
    l_lda.issue( l_ra, l_st, l_wave, l_t * BK, l_K, uint32_t( l_t ) * l_kb_a );
    l_ldb.issue( l_rb, l_st + SA, l_wave, l_t * BK, l_K, uint32_t( l_t ) * l_kb_b );
  }
}

// Main loop after the prologue's loads were issued.  FIRST_VMCNT: what may
// still be in flight beyond the prologue's loads when the loop starts
//   -1: nothing; the waits count only the loads issued after the awaited ones
//    0: unknown; the first wait is for everything, vmcnt(0)
//    1: when l_pend, at least 63 stores issued after the prologue (the
//       previous tile's output).  The waits for the prologue's steps (0 ..
//       STAGES-2) are then vmcnt(63): every one of those loads has at least
//       63 younger operations behind it, so at most 63 outstanding means it
//       has landed, while the stores keep draining under the first steps'
//       MFMAs (vmcnt counts loads and stores in one in-order counter).  The
//       first wait for a load issued inside the loop, after the stores,
//       counts normally and so also waits for the stores.
// Ends after the last step's MFMAs are issued; the stage buffers may still
// be read by other waves.
template< int BM, int BN, int BK, int WM, int WN, int MA, int MB, int STAGES, int FIRST_VMCNT,
          typename LdA, typename LdB, typename FrA, typename FrB, int TM, int TN >
__device__ __attribute__( ( always_inline ) ) inline void mainloop_body(
    f32x16 ( &l_acc )[TM][TN], char * l_lds, LdA & l_lda, LdB & l_ldb, FrA const & l_fra, FrB const & l_frb,
    i32x4 l_ra, i32x4 l_rb, int l_wave, int32_t l_K, int32_t l_nk, uint32_t l_kb_a, uint32_t l_kb_b,
    bool l_pend = false ) {
  constexpr int SA  = LdA::STAGE_BYTES;
  constexpr int SB  = LdB::STAGE_BYTES;
  constexpr int NJA = LdA::NJ;
  constexpr int NJW = LdA::NJ + LdB::NJ;
  constexpr int NMF = TM * TN;
  constexpr int PB  = 4;                           // MFMAs before the barrier
  typedef ReadOrder< TM, TN, FrA::UNITS, FrB::UNITS > RO;
  constexpr int U   = RO::U;
  constexpr MfmaOrder< TM, TN > kMo{};
  constexpr RO kRo{};
  static_assert( STAGES >= 3, "loads run at least two steps ahead" );
  static_assert( NJW <= 2 * NMF, "at most one DMA issue per MFMA" );
  // DMA issue d sits after MFMA dma_slot(d) of the step (MFMA index over both
  // substeps, evenly spread), after any wait at that MFMA; the wait + barrier
  // sit after MFMA NMF + PB - 1.  DMA_BEFORE = issues of this step before it.
  constexpr int DMA_BEFORE = dma_before< 2 * NMF, NJW >( NMF + PB - 1 );

  uint32_t const l_lds0 = lds_addr( l_lds );
  typename FrA::Part l_pa[2][TM];
  typename FrB::Part l_pb[2][TN];

  // step 0 has landed, then fragments of step 0, substep 0
  if constexpr( FIRST_VMCNT < 0 ) wait_vmcnt< ( STAGES - 2 ) * NJW >();
  else if constexpr( FIRST_VMCNT == 0 ) wait_vmcnt< 0 >();
  else {
    if( l_pend ) wait_vmcnt< 63 >();
    else         wait_vmcnt< ( STAGES - 2 ) * NJW >();
  }
  barrier_lds();
  static_for< U >( [&]( auto rc ) __attribute__( ( always_inline ) ) {
    constexpr int l_r = decltype( rc )::value;
    if constexpr( kRo.isb[l_r] == 0 ) l_fra.template read_unit< kRo.unit[l_r] >( l_lds, kRo.idx[l_r], 0, l_pa[0][kRo.idx[l_r]] );
    else l_frb.template read_unit< kRo.unit[l_r] >( l_lds + SA, kRo.idx[l_r], 0, l_pb[0][kRo.idx[l_r]] );
  } );

  // M0 of this wave's first DMA chunk in stage 0, per operand
  uint32_t const l_m0a = l_lds0 + uint32_t( l_wave * LdA::NJ * 1024 );
  uint32_t const l_m0b = l_lds0 + uint32_t( SA + l_wave * LdB::NJ * 1024 );

  // ST >= 0: t % STAGES == ST known at compile time (stage offsets become
  // instruction immediates); ST < 0: computed
  // FG: 1 = the first STAGES steps (compile-time ST), 0 = a later group of
  // them, -1 = unknown (checked at run time)
  auto iteration = [&]( int32_t l_t, auto dma_c, auto next_c, auto chk_c, auto st_c, auto fg_c ) __attribute__( ( always_inline ) ) {
    constexpr bool DMA  = decltype( dma_c )::value;
    constexpr bool NEXT = decltype( next_c )::value;
    constexpr bool CHK  = decltype( chk_c )::value;
    constexpr int  ST   = decltype( st_c )::value;
    constexpr int  FG   = decltype( fg_c )::value;
    constexpr int  OFF_CUR = ( ST >= 0 ? ST : 0 ) * ( SA + SB );
    constexpr int  OFF_NXT = ( ST >= 0 ? ( ST + 1 ) % STAGES : 0 ) * ( SA + SB );
    int32_t const l_cs = ( ST >= 0 ) ? ST : l_t % STAGES;
    int32_t const l_ns = ( ST >= 0 ) ? ( ST + 1 ) % STAGES : ( l_t + 1 ) % STAGES;
    int32_t const l_ds = ( ST >= 0 ) ? ( ST + STAGES - 1 ) % STAGES : ( l_t + STAGES - 1 ) % STAGES;
    char const * l_sa = l_lds + l_cs * ( SA + SB );
    char const * l_sb = l_sa + SA;
    char const * l_na = l_lds + l_ns * ( SA + SB );
    int32_t const l_tl = l_t + STAGES - 1;
    uint32_t const l_soa = uint32_t( l_tl ) * l_kb_a;
    uint32_t const l_sob = uint32_t( l_tl ) * l_kb_b;

    // both substeps as one sequence of 2 * NMF MFMAs; DMA issues spread
    // evenly over it (one per 2 * NMF / NJW MFMAs) so the address unit is
    // never asked for a whole step's loads at once
    static_for< 2 * NMF >( [&]( auto qc ) __attribute__( ( always_inline ) ) {
      constexpr int l_q = decltype( qc )::value;
      constexpr int l_s = l_q / NMF;                 // substep
      constexpr int l_p = l_q % NMF;                 // MFMA within the substep
      constexpr int l_i = kMo.i[l_p];
      constexpr int l_j = kMo.j[l_p];
      l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16( FrA::value( l_pa[l_s][l_i] ),
                                                                 FrB::value( l_pb[l_s][l_j] ),
                                                                 l_acc[l_i][l_j], 0, 0, 0 );
      if constexpr( l_s == 0 ) {
        // fragments of substep 1 of this step
        static_for< U >( [&]( auto rc ) __attribute__( ( always_inline ) ) {
          constexpr int l_r = decltype( rc )::value;
          if constexpr( ( l_r * NMF ) / U == l_p ) {
            if constexpr( ST >= 0 ) {
              if constexpr( kRo.isb[l_r] == 0 )
                l_fra.template read_unit_c< kRo.unit[l_r], OFF_CUR + 16 * BM * 2 >( l_lds, kRo.idx[l_r], l_pa[1][kRo.idx[l_r]] );
              else
                l_frb.template read_unit_c< kRo.unit[l_r], OFF_CUR + SA + 16 * BN * 2 >( l_lds, kRo.idx[l_r], l_pb[1][kRo.idx[l_r]] );
            }
            else if constexpr( kRo.isb[l_r] == 0 )
              l_fra.template read_unit< kRo.unit[l_r] >( l_sa, kRo.idx[l_r], 1, l_pa[1][kRo.idx[l_r]] );
            else
              l_frb.template read_unit< kRo.unit[l_r] >( l_sb, kRo.idx[l_r], 1, l_pb[1][kRo.idx[l_r]] );
          }
        } );
      }
      else if constexpr( NEXT ) {
        if constexpr( l_p == PB - 1 ) {
          // step t + 1 is complete once at most the loads issued after it
          // are in flight: all of steps t + 2 .. t + STAGES - 2 (issued in
          // earlier steps) and the DMA_BEFORE loads of step t + STAGES - 1
          // issued so far in this step
          // (with FIRST_VMCNT 1 and l_pend, the prologue's steps have the
          // previous tile's stores behind them: vmcnt(63), see above; FG
          // says whether this is such a step at compile time)
          auto wait_normal = [&]() __attribute__( ( always_inline ) ) {
            if constexpr( DMA ) wait_vmcnt< ( STAGES - 3 ) * NJW + DMA_BEFORE >();
            else                wait_vmcnt< 0 >();
          };
          if constexpr( FG == 0 || FIRST_VMCNT != 1 ) wait_normal();
          else if constexpr( FG == 1 ) {
            if constexpr( ST + 1 <= STAGES - 2 ) {
              if( l_pend ) wait_vmcnt< 63 >();
              else wait_normal();
            }
            else wait_normal();
          }
          else if( l_pend && l_t + 1 <= STAGES - 2 ) wait_vmcnt< 63 >();
          else wait_normal();
          wait_lgkmcnt0();
          barrier_lds();
        }
        // fragments of substep 0 of step t + 1
        static_for< U >( [&]( auto rc ) __attribute__( ( always_inline ) ) {
          constexpr int l_r = decltype( rc )::value;
          if constexpr( l_p >= PB && PB + ( l_r * ( NMF - PB ) ) / U == l_p ) {
            if constexpr( ST >= 0 ) {
              if constexpr( kRo.isb[l_r] == 0 )
                l_fra.template read_unit_c< kRo.unit[l_r], OFF_NXT >( l_lds, kRo.idx[l_r], l_pa[0][kRo.idx[l_r]] );
              else
                l_frb.template read_unit_c< kRo.unit[l_r], OFF_NXT + SA >( l_lds, kRo.idx[l_r], l_pb[0][kRo.idx[l_r]] );
            }
            else if constexpr( kRo.isb[l_r] == 0 )
              l_fra.template read_unit< kRo.unit[l_r] >( l_na, kRo.idx[l_r], 0, l_pa[0][kRo.idx[l_r]] );
            else
              l_frb.template read_unit< kRo.unit[l_r] >( l_na + SA, kRo.idx[l_r], 0, l_pb[0][kRo.idx[l_r]] );
          }
        } );
      }
      if constexpr( DMA ) {
        static_for< NJW >( [&]( auto dc ) __attribute__( ( always_inline ) ) {
          constexpr int l_d = decltype( dc )::value;
          if constexpr( dma_slot< 2 * NMF, NJW >( l_d ) == l_q ) {
            if constexpr( l_d == 0 || l_d == NJA ) {
              uint32_t const l_base = ( l_d == 0 ) ? l_m0a : l_m0b;
              if constexpr( ST >= 0 ) set_m0_add< uint32_t( ( ( ST + STAGES - 1 ) % STAGES ) * ( SA + SB ) ) >( l_base );
              else set_m0( l_base + uint32_t( l_ds ) * ( SA + SB ) );
            }
            if constexpr( l_d < NJA )
              l_lda.template issue_so< l_d, CHK >( l_ra, l_soa, l_tl * BK, l_K );
            else
              l_ldb.template issue_so< l_d - NJA, CHK >( l_rb, l_sob, l_tl * BK, l_K );
          }
        } );
      }
      __builtin_amdgcn_sched_barrier( 0 );
    } );
  };

  std::integral_constant< bool, true >  const l_yes{};
  std::integral_constant< bool, false > const l_no{};
  std::integral_constant< int, -1 > const l_rt{};
  std::integral_constant< int, 1 > const l_fg1{};
  std::integral_constant< int, 0 > const l_fg0{};
  int32_t l_t = 0;
  // steps whose loads (step t + STAGES - 1 < nk - 1) are whole k steps, in
  // groups of STAGES with compile-time stage indices (the first group, where
  // the previous tile's stores may still be pending, separately)
  if( l_nk - STAGES >= STAGES ) {
    static_for< STAGES >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
      iteration( decltype( sc )::value, l_yes, l_yes, l_no, sc, l_fg1 );
    } );
    for( l_t = STAGES; l_t + STAGES <= l_nk - STAGES; l_t += STAGES ) {
      static_for< STAGES >( [&]( auto sc ) __attribute__( ( always_inline ) ) {
        iteration( l_t + decltype( sc )::value, l_yes, l_yes, l_no, sc, l_fg0 );
      } );
    }
  }
  // (an early return or a conditional last step here made the compiler
  // spill the accumulators)
  for( ; l_t < l_nk - STAGES; l_t++ ) iteration( l_t, l_yes, l_yes, l_no, l_rt, l_rt );
  for( ; l_t < l_nk - ( STAGES - 1 ); l_t++ ) iteration( l_t, l_yes, l_yes, l_yes, l_rt, l_rt );
  for( ; l_t < l_nk - 1; l_t++ ) iteration( l_t, l_no, l_yes, l_yes, l_rt, l_rt );
  iteration( l_nk - 1, l_no, l_no, l_yes, l_rt, l_rt );
}

template< int BM, int BN, int BK, int WM, int WN, int MA, int MB, int STAGES, typename LdA, typename LdB,
          typename FrA, typename FrB, int TM, int TN >
__device__ __attribute__( ( always_inline ) ) inline void mainloop_scheduled(
    f32x16 ( &l_acc )[TM][TN], char * l_lds, LdA & l_lda, LdB & l_ldb, FrA const & l_fra, FrB const & l_frb,
    i32x4 l_ra, i32x4 l_rb, int l_wave, int32_t l_K, int32_t l_nk, uint32_t l_kb_a, uint32_t l_kb_b ) {
  prologue_issue< BK, STAGES >( l_lds, l_lda, l_ldb, l_ra, l_rb, l_wave, l_K, l_kb_a, l_kb_b );
  mainloop_body< BM, BN, BK, WM, WN, MA, MB, STAGES, -1 >( l_acc, l_lds, l_lda, l_ldb, l_fra, l_frb, l_ra,
                                                                l_rb, l_wave, l_K, l_nk, l_kb_a, l_kb_b );
  // the prologue's loads past the last step (zeros) still target LDS: drain
  // them before the epilogue reuses it
  wait_vmcnt< 0 >();
  barrier_lds();
}

// ---------------------------------------------------------------------------
// tile order: linear tile id -> (c, first row, first column).  C outermost
// (or innermost for c_inner), and within one C index groups of 8 tile rows
// walked column by column, so the workgroups running side by side on one XCD
// share their A rows and B columns in that XCD's L2.
// ---------------------------------------------------------------------------
template< int BM, int BN >
__device__ inline void decode_tile( ContractArgs const & a, int32_t l_lin, int32_t & o_c, int32_t & o_m0,
                                    int32_t & o_n0 ) {
  int32_t const l_ntiles = a.tiles_m * a.tiles_n;
  int32_t const l_c      = a.c_inner ? l_lin % a.C : l_lin / l_ntiles;
  int32_t const l_tile   = a.c_inner ? l_lin / a.C : l_lin - l_c * l_ntiles;
  constexpr int32_t kGroupM = 8;
  int32_t const l_in_grp = kGroupM * a.tiles_n;
  int32_t const l_grp    = l_tile / l_in_grp;
  int32_t const l_fm     = l_grp * kGroupM;
  int32_t const l_gsz    = min( a.tiles_m - l_fm, kGroupM );
  int32_t const l_tm     = l_fm + ( l_tile - l_grp * l_in_grp ) % l_gsz;
  int32_t const l_tn     = ( l_tile - l_grp * l_in_grp ) / l_gsz;
  o_c  = l_c;
  o_m0 = l_tm * BM;
  o_n0 = l_tn * BN;
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
template< int BM, int BN, int BK, int WM, int WN, int MA, int MB, int STAGES, int WPE = 1 >
__global__ __launch_bounds__( 64 * WM * WN, WPE )
void contract_dma_kernel( ContractArgs a ) {
  constexpr int W   = WM * WN;
  constexpr int T   = 64 * W;
  constexpr int TM  = BM / WM / 32;
  constexpr int TN  = BN / WN / 32;
  constexpr int SUB = BK / 16;
  typedef DmaLoader< BM, BK, W, MA > LdA;
  typedef DmaLoader< BN, BK, W, MB > LdB;
  constexpr int SA  = LdA::STAGE_BYTES;
  constexpr int SB  = LdB::STAGE_BYTES;
  constexpr int NJW = LdA::NJ + LdB::NJ;     // DMA instructions per wave and stage
  static_assert( STAGES >= 2, "at least double buffering" );
  static_assert( ( STAGES - 2 ) * NJW < 64, "vmcnt range" );

  __shared__ __attribute__( ( aligned( 1024 ) ) ) char l_lds[STAGES * ( SA + SB )];

  // tile order: see contract_kernel (XCD-contiguous ranges, groups of 8 tile rows)
  int32_t const l_nblk = gridDim.x;
  int32_t l_bid = blockIdx.x;
  if( ( l_nblk & 7 ) == 0 ) l_bid = ( l_bid & 7 ) * ( l_nblk >> 3 ) + ( l_bid >> 3 );
  int32_t l_c, l_m0, l_n0;
  decode_tile< BM, BN >( a, l_bid, l_c, l_m0, l_n0 );

  int const l_lane = threadIdx.x & 63;
  int const l_wave = __builtin_amdgcn_readfirstlane( threadIdx.x >> 6 );
  int const l_wm   = l_wave / WN;
  int const l_wn   = l_wave - l_wm * WN;

  uint16_t const * l_pa = reinterpret_cast< uint16_t const * >( a.a ) + a.tc_a[l_c];
  uint16_t const * l_pb = reinterpret_cast< uint16_t const * >( a.b ) + a.tc_b[l_c];
  i32x4 const l_ra = make_rsrc( l_pa, kDmaOob );
  i32x4 const l_rb = make_rsrc( l_pb, kDmaOob );

  LdA l_lda;
  LdB l_ldb;
  l_lda.init( a.tm_a, a.M, l_m0, a.sk_a, l_wave, l_lane );
  l_ldb.init( a.tn_b, a.N, l_n0, a.sk_b, l_wave, l_lane );

  DmaFrag< BM, BK, TM, MA > l_fra;
  DmaFrag< BN, BK, TN, MB > l_frb;
  l_fra.init( l_wm * TM * 32, l_lane );
  l_frb.init( l_wn * TN * 32, l_lane );
  if constexpr( MA == LOAD_VEC_MN ) l_fra.init_hi();
  if constexpr( MB == LOAD_VEC_MN ) l_frb.init_hi();

  f32x16 l_acc[TM][TN];
#pragma unroll
  for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
    for( int l_j = 0; l_j < TN; l_j++ )
      l_acc[l_i][l_j] = f32x16( 0.0f );

  int32_t const l_K  = a.K;
  int32_t const l_nk = ( l_K + BK - 1 ) / BK;
  uint32_t const l_kb_a = uint32_t( 2 * BK * a.sk_a );   // bytes per k step
  uint32_t const l_kb_b = uint32_t( 2 * BK * a.sk_b );
  uint32_t const l_lds0 = lds_addr( l_lds );

  if constexpr( SUB == 2 && STAGES >= 3 ) {
    if( l_nk > 0 ) {
      mainloop_scheduled< BM, BN, BK, WM, WN, MA, MB, STAGES >( l_acc, l_lds, l_lda, l_ldb, l_fra, l_frb, l_ra,
                                                                l_rb, l_wave, l_K, l_nk, l_kb_a, l_kb_b );
    }
  }
  else if( l_nk > 0 ) {
    // prologue: steps 0 .. STAGES-2 (steps >= nk load zeros)
#pragma unroll
    for( int l_t = 0; l_t < STAGES - 1; l_t++ ) {
      uint32_t const l_st = l_lds0 + uint32_t( l_t ) * ( SA + SB );
      l_lda.issue( l_ra, l_st, l_wave, l_t * BK, l_K, uint32_t( l_t ) * l_kb_a );
      l_ldb.issue( l_rb, l_st + SA, l_wave, l_t * BK, l_K, uint32_t( l_t ) * l_kb_b );
    }
    wait_vmcnt< ( STAGES - 2 ) * NJW >();
    barrier_lds();

    bf16x8 l_fa[2][TM];
    bf16x8 l_fb[2][TN];
#pragma unroll
    for( int l_i = 0; l_i < TM; l_i++ ) l_fa[0][l_i] = l_fra.read( l_lds, l_i, 0 );
#pragma unroll
    for( int l_j = 0; l_j < TN; l_j++ ) l_fb[0][l_j] = l_frb.read( l_lds + SA, l_j, 0 );

    for( int32_t l_t = 0; l_t < l_nk; l_t++ ) {
      // loads for step t + STAGES - 1 go into the buffer of step t - 1, which
      // every wave finished reading before the barrier that ended step t - 1
      {
        int32_t const l_tl = l_t + STAGES - 1;
        uint32_t const l_st = l_lds0 + uint32_t( l_tl % STAGES ) * ( SA + SB );
        l_lda.issue( l_ra, l_st, l_wave, l_tl * BK, l_K, uint32_t( l_tl ) * l_kb_a );
        l_ldb.issue( l_rb, l_st + SA, l_wave, l_tl * BK, l_K, uint32_t( l_tl ) * l_kb_b );
      }
      char const * l_sa = l_lds + ( l_t % STAGES ) * ( SA + SB );
      char const * l_sb = l_sa + SA;
#pragma unroll
      for( int l_s = 0; l_s < SUB; l_s++ ) {
        int const l_cur = l_s & 1;
        int const l_nxt = l_cur ^ 1;
        if( l_s + 1 < SUB ) {
#pragma unroll
          for( int l_i = 0; l_i < TM; l_i++ ) l_fa[l_nxt][l_i] = l_fra.read( l_sa, l_i, l_s + 1 );
#pragma unroll
          for( int l_j = 0; l_j < TN; l_j++ ) l_fb[l_nxt][l_j] = l_frb.read( l_sb, l_j, l_s + 1 );
        }
        else if( l_t + 1 < l_nk ) {
          // step t + 1 must have landed (own loads: vmcnt; everyone's: barrier)
          wait_vmcnt< ( STAGES - 2 ) * NJW >();
          wait_lgkmcnt0();                    // this step's LDS reads are done
          barrier_lds();
          char const * l_na = l_lds + ( ( l_t + 1 ) % STAGES ) * ( SA + SB );
#pragma unroll
          for( int l_i = 0; l_i < TM; l_i++ ) l_fa[l_nxt][l_i] = l_fra.read( l_na, l_i, 0 );
#pragma unroll
          for( int l_j = 0; l_j < TN; l_j++ ) l_fb[l_nxt][l_j] = l_frb.read( l_na + SA, l_j, 0 );
        }
#pragma unroll
        for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
          for( int l_j = 0; l_j < TN; l_j++ )
            l_acc[l_i][l_j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16( l_fa[l_cur][l_i], l_fb[l_cur][l_j],
                                                                       l_acc[l_i][l_j], 0, 0, 0 );
      }
    }
    // the trailing (zero) loads still target LDS: drain them before the
    // epilogue reuses it
    wait_vmcnt< 0 >();
    barrier_lds();
  }

  static_assert( EpilogueLds< BM, BN, WM, WN, TM, TN >::BYTES <= int( sizeof( l_lds ) ),
                 "LDS too small for the epilogue" );
  // the offset tables are read here, not at the start: the main loop holds
  // no registers for them
  EpilogueTabs< BM, BN, T > l_tabs;
  l_tabs.load( a, l_m0, l_n0 );
  epilogue< BM, BN, WM, WN, TM, TN, T >( a, l_acc, l_tabs, l_lds, l_c, l_m0, l_n0, l_wm, l_wn, l_lane );
}


// ---------------------------------------------------------------------------
// Persistent variant (VEC_MN x VEC_MN, scheduled BK 32 loop): one workgroup
// per CU walks its share of the tiles.  Per tile it
//   * reads the NEXT task's loader offsets and epilogue tables (global loads
//     that land during this tile's main loop),
//   * runs the main loop,
//   * issues the next task's first STAGES-1 k-steps before its own output
//     stores (the loads land while the stores drain; the epilogue's tables
//     live in their own LDS region), then stores the output.
// Tiles are split into XCD-contiguous ranges exactly as in the one-tile-per-
// workgroup kernel (workgroup w runs on XCD w % 8 and takes every
// (gridDim / 8)-th tile of XCD w % 8's range), so the L2 sharing is the same.
//
// Staggered start (dma_phases P > 1): workgroup w waits (w / 8) % P times
// dma_stagger sleep units of about 1 us before its first tile.  Workgroups
// that finish their tiles at the same moment store at the same moment, and
// the 32 CUs of one XCD storing 256 KB each at once are bounded by that
// XCD's share of the write bandwidth while their matrix cores idle; with the
// phases offset, part of one phase's stores overlap another's main loop.
// (Offsets between whole XCDs do not help: each XCD's own write path is the
// bound.)
//
// Runs only contractions whose tiles are all full and take the plain fast
// epilogue with non-temporal stores: fp32 output, 32-bit output offsets,
// output columns in unit-stride runs of 32, ZERO first touch, no last touch
// (persistent_dma_eligible; a second store variant in the kernel makes the
// compiler copy the accumulators into VGPRs); the others use
// contract_dma_kernel.
// ---------------------------------------------------------------------------
__host__ __device__ inline bool persistent_dma_eligible( ContractArgs const & a, int BM, int BN ) {
  return a.M % BM == 0 && a.N % BN == 0 && a.out_off32 && a.out_nt && !a.out_bf16
      && a.first_touch == ETIR_KTYPE_ZERO && a.last_touch == ETIR_KTYPE_UNDEFINED;
}

template< int BM, int BN, int BK, int WM, int WN, int STAGES >
__global__ __launch_bounds__( 64 * WM * WN, 1 )
void contract_dma_persistent_kernel( ContractArgs a ) {
  constexpr int MA  = LOAD_VEC_MN;
  constexpr int MB  = LOAD_VEC_MN;
  constexpr int W   = WM * WN;
  constexpr int T   = 64 * W;
  constexpr int TM  = BM / WM / 32;
  constexpr int TN  = BN / WN / 32;
  typedef DmaLoader< BM, BK, W, MA > LdA;
  typedef DmaLoader< BN, BK, W, MB > LdB;
  typedef EpilogueTabs< BM, BN, T > Tabs;
  constexpr int SA  = LdA::STAGE_BYTES;
  constexpr int SB  = LdB::STAGE_BYTES;
  constexpr int OPS = STAGES * ( SA + SB );              // operand stage buffers
  constexpr int TABS = EpilogueLds< BM, BN, WM, WN, TM, TN >::TABS;
  static_assert( BK == 32 && STAGES >= 3, "persistent kernel runs the scheduled BK 32 loop" );
  static_assert( 16 * TM * TN >= 63, "vmcnt(63) waits need 63 stores behind the prologue" );

  __shared__ __attribute__( ( aligned( 1024 ) ) ) char l_lds[OPS + TABS];
  int32_t * l_tabs_lds = reinterpret_cast< int32_t * >( l_lds + OPS );

  // this workgroup's tiles: linear ids l_first, l_first + l_step, ... < l_end
  int32_t const l_ntiles_all = a.C * a.tiles_m * a.tiles_n;
  int32_t const l_nwg = gridDim.x;
  int32_t l_first, l_step, l_end;
  if( ( l_nwg & 7 ) == 0 && ( l_ntiles_all & 7 ) == 0 ) {
    int32_t const l_x  = blockIdx.x & 7;
    int32_t const l_t8 = l_ntiles_all >> 3;
    l_first = l_x * l_t8 + ( blockIdx.x >> 3 );
    l_step  = l_nwg >> 3;
    l_end   = ( l_x + 1 ) * l_t8;
  }
  else {
    l_first = blockIdx.x;
    l_step  = l_nwg;
    l_end   = l_ntiles_all;
  }
  if( l_first >= l_end ) return;
  int32_t const l_ntiles = ( l_end - l_first + l_step - 1 ) / l_step;

  int const l_lane = threadIdx.x & 63;
  int const l_wave = __builtin_amdgcn_readfirstlane( threadIdx.x >> 6 );
  int const l_wm   = l_wave / WN;
  int const l_wn   = l_wave - l_wm * WN;

  if( a.dma_phases > 1 ) {
    int32_t const l_ph = ( blockIdx.x >> 3 ) % a.dma_phases;
    for( int32_t l_z = 0; l_z < l_ph * a.dma_stagger; l_z++ ) __builtin_amdgcn_s_sleep( 32 );
  }

  DmaFrag< BM, BK, TM, MA > l_fra;
  DmaFrag< BN, BK, TN, MB > l_frb;
  l_fra.init( l_wm * TM * 32, l_lane );
  l_frb.init( l_wn * TN * 32, l_lane );
  if constexpr( MA == LOAD_VEC_MN ) l_fra.init_hi();
  if constexpr( MB == LOAD_VEC_MN ) l_frb.init_hi();

  int32_t const l_K  = a.K;
  int32_t const l_nk = ( l_K + BK - 1 ) / BK;
  uint32_t const l_kb_a = uint32_t( 2 * BK * a.sk_a );
  uint32_t const l_kb_b = uint32_t( 2 * BK * a.sk_b );
  uint16_t const * l_pa0 = reinterpret_cast< uint16_t const * >( a.a );
  uint16_t const * l_pb0 = reinterpret_cast< uint16_t const * >( a.b );

  int32_t const l_ntasks = l_ntiles;
  auto task_tile = [&]( int32_t t ) { return l_first + t * l_step; };

  // current task
  int32_t l_c, l_m0, l_n0;
  decode_tile< BM, BN >( a, task_tile( 0 ), l_c, l_m0, l_n0 );
  LdA l_lda;
  LdB l_ldb;
  l_lda.init( a.tm_a, a.M, l_m0, a.sk_a, l_wave, l_lane );
  l_ldb.init( a.tn_b, a.N, l_n0, a.sk_b, l_wave, l_lane );
  i32x4 l_ra = make_rsrc( l_pa0 + a.tc_a[l_c], kDmaOob );
  i32x4 l_rb = make_rsrc( l_pb0 + a.tc_b[l_c], kDmaOob );
  Tabs l_tabs;
  l_tabs.load( a, l_m0, l_n0 );
  prologue_issue< BK, STAGES >( l_lds, l_lda, l_ldb, l_ra, l_rb, l_wave, l_K, l_kb_a, l_kb_b );

  for( int32_t l_t = 0; l_t < l_ntasks; l_t++ ) {
    bool const l_has_next = l_t + 1 < l_ntasks;

    // the next task's offsets: read now, used after this task's main loop
    int32_t l_nc = l_c, l_nm0 = l_m0, l_nn0 = l_n0;
    LdA l_nlda = l_lda;
    LdB l_nldb = l_ldb;
    Tabs l_ntabs = l_tabs;
    if( l_has_next ) {
      // loads only: their values are first used after the main loop, so
      // nothing waits for them (or for the stores issued before them) here
      decode_tile< BM, BN >( a, task_tile( l_t + 1 ), l_nc, l_nm0, l_nn0 );
      l_nlda.load_rows( a.tm_a, a.M, l_nm0, l_wave, l_lane );
      l_nldb.load_rows( a.tn_b, a.N, l_nn0, l_wave, l_lane );
      l_ntabs.load( a, l_nm0, l_nn0 );
    }

    f32x16 l_acc[TM][TN];
#pragma unroll
    for( int l_i = 0; l_i < TM; l_i++ )
#pragma unroll
      for( int l_j = 0; l_j < TN; l_j++ )
        l_acc[l_i][l_j] = f32x16( 0.0f );
    if( l_nk > 0 ) {
      // the previous task's output stores (from the second task on) were
      // issued after this task's prologue loads
      mainloop_body< BM, BN, BK, WM, WN, MA, MB, STAGES, 1 >( l_acc, l_lds, l_lda, l_ldb, l_fra, l_frb, l_ra, l_rb,
                                                             l_wave, l_K, l_nk, l_kb_a, l_kb_b, l_t > 0 );
    }
    // every wave is done with the operand buffers (and nothing of this task
    // is still loading into them)
    wait_vmcnt< 0 >();
    wait_lgkmcnt0();
    barrier_lds();

    if( l_has_next ) {
      l_nlda.finalize( a.sk_a );
      l_nldb.finalize( a.sk_b );
    }
    i32x4 const l_nra = make_rsrc( l_pa0 + a.tc_a[l_nc], kDmaOob );
    i32x4 const l_nrb = make_rsrc( l_pb0 + a.tc_b[l_nc], kDmaOob );
    if( l_has_next ) {
      prologue_issue< BK, STAGES >( l_lds, l_nlda, l_nldb, l_nra, l_nrb, l_wave, l_K, l_kb_a, l_kb_b );
    }
    l_tabs.stage( l_tabs_lds );
    wait_lgkmcnt0();
    barrier_lds();
    {
      float * l_base = reinterpret_cast< float * >( a.out ) + a.tc_out[l_c];
      int const l_row0 = l_wm * TM * 32;
      int const l_col0 = l_wn * TN * 32;
      int32_t const * l_so_m = l_tabs_lds;
      int32_t const * l_so_n = l_tabs_lds + 2 * BM;
      epilogue_fast_f32< TM, TN, false >( l_base, l_acc, l_so_m, l_so_n, l_row0, l_col0, l_lane );
      // the staged tables are rewritten at the next task's epilogue, a whole
      // main loop (and its barriers) later
    }

    l_c = l_nc;
    l_m0 = l_nm0;
    l_n0 = l_nn0;
    l_lda = l_nlda;
    l_ldb = l_nldb;
    l_tabs = l_ntabs;
    l_ra = l_nra;
    l_rb = l_nrb;
  }
  // nothing may still write LDS when the workgroup ends
  wait_vmcnt< 0 >();
}

}  // namespace kern
}  // namespace etir

#endif
