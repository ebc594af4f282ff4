// fp32 contractions with a short K (at most 64) and one free side of 65 to
// 256 against a long other side:
//   out[m][n] = touch( sum_k A[m][k] * B[n][k] ).
//
// On the MFMA tiles such a node spends each tile in one load round trip and
// its stores, and pads K to the tile's k step (the einsum_benchmark MERA
// root, M = 177147, N = 243, K = 50: 74 us on 128 x 128 tiles for 172 MB of
// output that a plain fill writes in 26 us).  Here one persistent workgroup
// of 8 waves per CU
//   * keeps the short operand in LDS for the whole launch ([k][s], read once
//     through its offset tables),
//   * walks panels of the long side (64 rows with a short side of up to 256,
//     128 rows up to 128), each panel prefetched into registers one panel
//     ahead and written to LDS when the previous one is done,
//   * computes a panel with v_mfma_f32_32x32x2f32 over exactly ceil(K / 2)
//     k pairs (each wave a 32 x 64 block: one 32-block of the panel, two of
//     the short side),
//   * and stores the previous panel's results between the MFMAs of the
//     current one, so the output writes run under the matrix work.
// The stores always issue, masked by the buffer range check (an offset past
// the output's extent is dropped), so every panel carries the same number of
// vector-memory operations and the compiler's wait for the prefetched loads
// counts exactly the stores issued after them.
//
// Sums run over k in the MFMA's pair order in fp32, as on the other MFMA
// tiles.  First touch ZERO, last touch none or RELU, fp32 output (the touch
// semantics of reference src/basic/binary/ContractionBackendTpp.cpp:84-163);
// other touches, aux tensors and C dims take the tiled kernels.
#include "etir_internal.h"
#include "contract_kernel.h"

namespace etir {

namespace {

using kern::f32x16;

constexpr int kPnWaves   = 8;
constexpr int kPnThreads = 64 * kPnWaves;
constexpr int kPnKMax    = 64;      // k rows of the LDS operands
constexpr int kPnStores  = 32;      // stores per wave and panel (2 blocks x 16)
// byte offset of a masked store: at or past every output extent the planner admits
constexpr uint32_t kPnOob = 0xfffffff0u;

// SP: short side padded (128 or 256); RES_A: the short (resident) operand is
// kernel A (the short side is kernel M), else kernel B; LFAST: the long
// operand is unit-stride along the long side (panel loads walk it), else the
// loads walk K
//
// LDS layouts (k padded with zeros to KP = 4 ceil(K / 4)):
//   resident [k][s], pitch SP + 1;
//   panel: element (k, l) at row 2 (k / 4) + k % 2, column 2 l + (k / 2) % 2
//   (pitch 2 PL + 2), so that one 8-byte read gives a lane (l, h) its
//   values of k = 4 g + h and 4 g + 2 + h: the A/B operand of two
//   consecutive k pairs of v_mfma_f32_32x32x2f32 (lane (r, h) supplies row
//   r, k = 2 kp + h).
template< int SP, bool RES_A, bool RELU, bool LFAST >
__global__ __launch_bounds__( kPnThreads, 1 ) void contract_panel_kernel( ContractArgs a, int32_t n_panels ) {
  constexpr int PL  = 16384 / SP;                    // long-side rows per panel
  constexpr int NSG = SP / 64;                       // waves along the short side
  constexpr int NE  = PL * kPnKMax / kPnThreads;     // panel elements per thread (at K = 64)
  constexpr int NR  = SP * kPnKMax / kPnThreads;     // resident elements per thread (at K = 64)
  constexpr int RP  = SP + 1;
  constexpr int PQ  = 2 * PL + 2;
  constexpr int NG  = kPnKMax / 4;                   // groups of two k pairs
  static_assert( ( PL / 32 ) * NSG == kPnWaves, "one 32 x 64 block per wave" );
  __shared__ float s_res[kPnKMax * RP];
  __shared__ __attribute__( ( aligned( 16 ) ) ) float s_pan[2][2 * NG * PQ];
  __shared__ __attribute__( ( aligned( 16 ) ) ) int32_t s_res_off[SP];
  __shared__ __attribute__( ( aligned( 16 ) ) ) int32_t s_pan_off[3][PL];

  int const l_tid  = threadIdx.x;
  int const l_lane = l_tid & 63;
  int const l_wave = __builtin_amdgcn_readfirstlane( l_tid >> 6 );
  int const l_wl   = l_wave / NSG;
  int const l_ws   = l_wave - l_wl * NSG;
  int const l_r    = l_lane & 31;
  int const l_h    = l_lane >> 5;

  int32_t const l_S   = RES_A ? a.M : a.N;
  int32_t const l_L   = RES_A ? a.N : a.M;     // >= PL (launch-checked)
  int32_t const l_K   = a.K;
  int32_t const l_kp  = ( l_K + 3 ) & ~3;      // k rows in LDS, zeros from K on
  int32_t const l_ng  = l_kp >> 2;             // groups of two k pairs
  bool const    l_kaff = a.k_affine != 0;
  // e / KP for e < 2^26 as a multiply-high: KP <= 64, magic = ceil(2^32 / KP)
  uint32_t const l_mg = uint32_t( ( ( uint64_t( 1 ) << 32 ) + uint32_t( l_kp ) - 1 ) / uint32_t( l_kp ) );
  auto div_kp = [&]( int32_t l_e ) __attribute__( ( always_inline ) ) {
    return int32_t( __umulhi( uint32_t( l_e ), l_mg ) );
  };

  // ------------------------------------------ long operand: panel elements
  // element e = tid + 512 i of a panel is (l, k) = (e % PL, e / PL) when the
  // long side is unit-stride (LFAST), else (e / KP, e % KP)
  float const * l_lp = reinterpret_cast< float const * >( RES_A ? a.b : a.a ) + ( RES_A ? a.tc_b[0] : a.tc_a[0] );
  int32_t const l_sl = RES_A ? a.sn_b : a.sm_a;            // affine long-side stride (launch-checked)
  int32_t const * l_to_l = RES_A ? a.tn_out : a.tm_out;
  uint32_t l_goff[NE];                                     // offset from the panel's first row
  int32_t  l_pidx[NE];                                     // LDS index, -1: no element
  uint32_t l_zero = 0;                                     // bit i: element i is a k padding row
  {
    int32_t const * l_tk = RES_A ? a.tk_b : a.tk_a;
    int32_t const   l_sk = RES_A ? a.sk_b : a.sk_a;
    int32_t const l_n = PL * l_kp;
    kern::static_for< NE >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
      constexpr int l_i = decltype( ic )::value;
      int32_t const l_e = l_tid + kPnThreads * l_i;
      int32_t const l_q = div_kp( l_e );
      int32_t const l_l = l_e < l_n ? ( LFAST ? ( l_e & ( PL - 1 ) ) : l_q ) : 0;
      int32_t const l_k = LFAST ? l_e / PL : l_e - l_q * l_kp;
      int32_t const l_kc = min( l_k, l_K - 1 );
      l_goff[l_i] = uint32_t( l_l * l_sl ) + uint32_t( l_kaff ? l_kc * l_sk : l_tk[l_kc] );
      l_pidx[l_i] = l_e < l_n ? ( 2 * ( l_k >> 2 ) + ( l_k & 1 ) ) * PQ + 2 * l_l + ( ( l_k >> 1 ) & 1 ) : -1;
      if( l_k >= l_K ) l_zero |= 1u << l_i;
    } );
  }
  // first long-side row of panel p: the last panel is moved back to end at
  // the long side's end (its first rows repeat the previous panel's, same
  // values stored twice), so every row of every panel is inside the tensor
  auto panel_row0 = [&]( int32_t l_pi ) __attribute__( ( always_inline ) ) {
    return min( min( l_pi, n_panels - 1 ) * PL, l_L - PL );
  };
  // one panel's elements and (threads < PL) its rows' output offsets, into
  // registers; panels past the last one reload the last (values unused)
  auto load_panel = [&]( int32_t l_pi, float ( &l_v )[NE], int32_t & l_off ) __attribute__( ( always_inline ) ) {
    int32_t const l_l0 = panel_row0( l_pi );
    float const * l_base = l_lp + int64_t( l_l0 ) * l_sl;
    kern::static_for< NE >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
      constexpr int l_i = decltype( ic )::value;
      l_v[l_i] = l_base[l_goff[l_i]];
    } );
    l_off = l_to_l[l_l0 + ( l_tid & ( PL - 1 ) )];
  };
  auto put_panel = [&]( int l_buf, int l_obuf, float const ( &l_v )[NE], int32_t l_off ) __attribute__( ( always_inline ) ) {
    kern::static_for< NE >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
      constexpr int l_i = decltype( ic )::value;
      if( l_pidx[l_i] >= 0 ) s_pan[l_buf][l_pidx[l_i]] = ( ( l_zero >> l_i ) & 1u ) ? 0.0f : l_v[l_i];
    } );
    if( l_tid < PL ) s_pan_off[l_obuf][l_tid] = l_off;
  };

  // this workgroup's panels: blockIdx.x, blockIdx.x + gridDim.x, ...
  int32_t const l_np = ( n_panels - int32_t( blockIdx.x ) + int32_t( gridDim.x ) - 1 ) / int32_t( gridDim.x );
  auto panel_of = [&]( int32_t t ) { return int32_t( blockIdx.x ) + t * int32_t( gridDim.x ); };

  // ---------------------------------------------------------- prologue
  // Every load of the prologue is issued before any of them is waited for:
  // panels 0 and 1, the short side's output offsets, the resident operand
  // (its row and k offsets computed where affine, else read from the tables
  // first -- the only dependent round trip).
  float   l_p0[NE], l_pre[NE];
  int32_t l_off0, l_pre_off;
  load_panel( panel_of( 0 ), l_p0, l_off0 );
  load_panel( panel_of( 1 ), l_pre, l_pre_off );
  int32_t const * l_to_s = RES_A ? a.tm_out : a.tn_out;
  int32_t const l_res_out = l_to_s[min( l_tid & ( SP - 1 ), l_S - 1 )];
  {
    float const * l_p = reinterpret_cast< float const * >( RES_A ? a.a : a.b ) + ( RES_A ? a.tc_a[0] : a.tc_b[0] );
    int32_t const * l_ts = RES_A ? a.tm_a : a.tn_b;
    int32_t const   l_ss = RES_A ? a.sm_a : a.sn_b;          // affine stride, or -1
    int32_t const * l_tk = RES_A ? a.tk_a : a.tk_b;
    int32_t const   l_sk = RES_A ? a.sk_a : a.sk_b;
    bool const l_kfast = l_kaff && l_sk == 1;  // consecutive threads on consecutive k
    int32_t const l_n = SP * l_kp;
    // element e = tid + 512 i is (s, k) = (e / KP, e % KP) or (e % SP, e / SP)
    int32_t  l_idx[NR];
    uint32_t l_off[NR];
    uint32_t l_ok = 0;
    kern::static_for< NR >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
      constexpr int l_i = decltype( ic )::value;
      int32_t const l_e = l_tid + kPnThreads * l_i;
      int32_t const l_q = div_kp( l_e );
      int32_t const l_s = l_kfast ? l_q : ( l_e & ( SP - 1 ) );
      int32_t const l_k = l_kfast ? l_e - l_q * l_kp : l_e / SP;
      int32_t const l_sc = min( l_s, l_S - 1 );
      int32_t const l_kc = min( l_k, l_K - 1 );
      l_off[l_i] = uint32_t( l_ss >= 0 ? l_sc * l_ss : l_ts[l_sc] ) + uint32_t( l_kaff ? l_kc * l_sk : l_tk[l_kc] );
      l_idx[l_i] = l_e < l_n ? l_k * RP + l_s : -1;
      if( ( l_s < l_S ) & ( l_k < l_K ) ) l_ok |= 1u << l_i;
    } );
    float l_v[NR];
    kern::static_for< NR >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
      constexpr int l_i = decltype( ic )::value;
      l_v[l_i] = l_p[l_off[l_i]];
    } );
    kern::static_for< NR >( [&]( auto ic ) __attribute__( ( always_inline ) ) {
      constexpr int l_i = decltype( ic )::value;
      if( l_idx[l_i] >= 0 ) s_res[l_idx[l_i]] = ( ( l_ok >> l_i ) & 1u ) ? l_v[l_i] : 0.0f;
    } );
  }
  if( l_tid < SP ) s_res_off[l_tid] = l_res_out;
  put_panel( 0, 0, l_p0, l_off0 );
  // Nothing of the prologue stays in flight into the loop: the compiler's
  // waits are per register, and a prologue load still pending in a register
  // the loop reuses (the accumulators) would make every panel's first MFMA
  // wait for the stores issued before it (one counter for loads and stores).
  // vmcnt(0), expcnt/lgkmcnt unconstrained (gfx9 encoding).
  __builtin_amdgcn_s_waitcnt( 0x0f70 );
  __syncthreads();

  // this wave's resident operands for every k pair, in registers for the
  // whole launch
  float l_y[2][kPnKMax / 2];
  kern::static_for< kPnKMax / 2 >( [&]( auto kc ) __attribute__( ( always_inline ) ) {
    constexpr int l_q = decltype( kc )::value;
    l_y[0][l_q] = s_res[( 2 * l_q + l_h ) * RP + 64 * l_ws + l_r];
    l_y[1][l_q] = s_res[( 2 * l_q + l_h ) * RP + 64 * l_ws + 32 + l_r];
  } );
  // the short side's output offsets: RES_A: D rows 64 ws + 32 j + 8 g + 4 h
  // + e, read from LDS two at a time a group ahead of their stores (bit q
  // of l_sok: store q's row inside S); else D columns 64 ws + 32 j + r, two
  // values in registers
  typedef int32_t i32x2v __attribute__( ( ext_vector_type( 2 ) ) );
  auto short_row = []( int l_q, int l_ws_, int l_h_ ) {
    return 64 * l_ws_ + 32 * ( l_q / 16 ) + 8 * ( ( l_q % 16 ) / 4 ) + 4 * l_h_ + l_q % 4;
  };
  int32_t  l_so[2] = { 0, 0 };
  uint32_t l_sok = 0;
  if constexpr( RES_A ) {
#pragma unroll
    for( int l_q = 0; l_q < kPnStores; l_q++ ) if( short_row( l_q, l_ws, l_h ) < l_S ) l_sok |= 1u << l_q;
  }
  else {
#pragma unroll
    for( int l_j = 0; l_j < 2; l_j++ ) {
      int const l_c = 64 * l_ws + 32 * l_j + l_r;
      l_so[l_j] = s_res_off[l_c];
      if( l_c < l_S ) l_sok |= 1u << l_j;
    }
  }

  // ------------------------------------------------------------- output
  __amdgpu_buffer_rsrc_t const l_rs =
      __builtin_amdgcn_make_buffer_rsrc( kern::uniform_ptr( reinterpret_cast< float * >( a.out ) + a.tc_out[0] ),
                                         (short) 0, (int) a.out_bytes, 0x00020000 );
  // store q (block j = q / 16, accumulator element v = q % 16: g = v / 4,
  // e = v % 4) of a finished panel's accumulators l_prv; l_po: that panel's
  // long-side output offsets this lane needs (RES_A: one, its D column; else
  // the 16 of its D rows 32 wl + 8 g + 4 h + e); l_sr (RES_A): the
  // short-side row offsets of stores q & ~1 and q | 1; l_ok false masks
  // every store
  typedef int32_t i32x4v __attribute__( ( ext_vector_type( 4 ) ) );
  constexpr int NPO = RES_A ? 1 : 16;
  auto store_one = [&]( auto qc, f32x16 const ( &l_prv )[2], int32_t const ( &l_po )[NPO], i32x2v l_sr,
                        bool l_ok ) __attribute__( ( always_inline ) ) {
    constexpr int l_q = decltype( qc )::value;
    int32_t l_off;
    bool l_in;
    if constexpr( RES_A ) {
      l_off = l_sr[l_q & 1] + l_po[0];
      l_in  = ( l_sok >> l_q ) & 1u;
    }
    else {
      l_off = l_po[l_q % 16] + l_so[l_q / 16];
      l_in  = ( l_sok >> ( l_q / 16 ) ) & 1u;
    }
    float l_x = l_prv[l_q / 16][l_q % 16];
    if constexpr( RELU ) l_x = fmaxf( l_x, 0.0f );
    uint32_t const l_b = ( l_ok & l_in ) ? uint32_t( l_off ) * 4u : kPnOob;
    __builtin_amdgcn_raw_buffer_store_b32( __builtin_bit_cast( uint32_t, l_x ), l_rs, l_b, 0, 0 );
  };
  // short-side row offsets of stores 2 g and 2 g + 1 (RES_A)
  auto short_pair = [&]( int l_g ) __attribute__( ( always_inline ) ) {
    if constexpr( RES_A ) return *reinterpret_cast< i32x2v const * >( s_res_off + short_row( 2 * l_g, l_ws, l_h ) );
    else                  return i32x2v{ 0, 0 };
  };
  auto panel_offsets = [&]( int l_ob, int32_t ( &l_po )[NPO] ) __attribute__( ( always_inline ) ) {
    if constexpr( RES_A ) {
      l_po[0] = s_pan_off[l_ob][32 * l_wl + l_r];
    }
    else {
      kern::static_for< 4 >( [&]( auto gc ) __attribute__( ( always_inline ) ) {
        constexpr int l_g = decltype( gc )::value;
        i32x4v const l_ro = *reinterpret_cast< i32x4v const * >( &s_pan_off[l_ob][32 * l_wl + 8 * l_g + 4 * l_h] );
        kern::static_for< 4 >( [&]( auto ec ) __attribute__( ( always_inline ) ) {
          constexpr int l_e = decltype( ec )::value;
          l_po[4 * l_g + l_e] = l_ro[l_e];
        } );
      } );
    }
  };
  typedef float f32x2v __attribute__( ( ext_vector_type( 2 ) ) );

  // One panel: MFMAs into l_cur (fresh: the first k pair takes a zero
  // accumulator), the previous panel's results (l_prv, finished one panel
  // ago) stored between them, then the next panel staged and the one after
  // it loaded.  Two accumulator sets alternate, so a panel's results are
  // stored straight from the registers the MFMAs wrote.
  auto panel = [&]( int32_t l_t, f32x16 ( &l_cur )[2], f32x16 const ( &l_prv )[2] ) __attribute__( ( always_inline ) ) {
    int const l_buf = l_t & 1;
    float const * l_pan = s_pan[l_buf] + l_h * PQ + 2 * ( 32 * l_wl + l_r );
    // the previous panel's row offsets (offset buffer (t + 2) % 3; nothing
    // is stored in the first panel)
    int32_t l_po[NPO];
    panel_offsets( ( l_t + 2 ) % 3, l_po );
    bool const l_prev = l_t > 0;

    // the panel's k pairs, two per group: the operands of group g + 1 read
    // (into the other register pair, unconditionally: no register is
    // rewritten while an MFMA that reads it may be in flight) before the
    // MFMAs of group g, two of the previous panel's stores after
    f32x2v l_x[2];
    l_x[0] = *reinterpret_cast< f32x2v const * >( l_pan );
    i32x2v l_sr = short_pair( 0 );
    kern::static_for< NG >( [&]( auto gc ) __attribute__( ( always_inline ) ) {
      constexpr int l_g  = decltype( gc )::value;
      constexpr int l_gn = ( l_g + 1 < NG ) ? l_g + 1 : 0;   // after the last group: group 0 again, unused
      i32x2v const l_srn = short_pair( l_gn );
      l_x[( l_g + 1 ) & 1] = *reinterpret_cast< f32x2v const * >( l_pan + 2 * l_gn * PQ );
      if( l_g == 0 || l_g < l_ng ) {
        kern::static_for< 2 >( [&]( auto jc ) __attribute__( ( always_inline ) ) {
          constexpr int l_j = decltype( jc )::value;
          constexpr int l_q = 2 * l_g + l_j;                  // k pair
          kern::static_for< 2 >( [&]( auto bc ) __attribute__( ( always_inline ) ) {
            constexpr int l_b = decltype( bc )::value;
            f32x16 const l_c = ( l_q == 0 ) ? f32x16( 0.0f ) : l_cur[l_b];
            float const  l_xv = l_x[l_g & 1][l_j];
            if constexpr( RES_A ) l_cur[l_b] = __builtin_amdgcn_mfma_f32_32x32x2f32( l_y[l_b][l_q], l_xv, l_c, 0, 0, 0 );
            else                  l_cur[l_b] = __builtin_amdgcn_mfma_f32_32x32x2f32( l_xv, l_y[l_b][l_q], l_c, 0, 0, 0 );
          } );
        } );
      }
      store_one( std::integral_constant< int, 2 * l_g >(), l_prv, l_po, l_sr, l_prev );
      store_one( std::integral_constant< int, 2 * l_g + 1 >(), l_prv, l_po, l_sr, l_prev );
      l_sr = l_srn;
    } );

    // next panel into the other buffers (last read in panel t - 1, before
    // the barrier that ended it), the one after it into registers
    put_panel( l_buf ^ 1, ( l_t + 1 ) % 3, l_pre, l_pre_off );
    load_panel( panel_of( l_t + 2 ), l_pre, l_pre_off );
    __syncthreads();
  };
  auto last_stores = [&]( f32x16 const ( &l_prv )[2] ) __attribute__( ( always_inline ) ) {
    int32_t l_po[NPO];
    panel_offsets( ( l_np - 1 ) % 3, l_po );
    kern::static_for< kPnStores / 2 >( [&]( auto gc ) __attribute__( ( always_inline ) ) {
      constexpr int l_g = decltype( gc )::value;
      i32x2v const l_sr = short_pair( l_g );
      store_one( std::integral_constant< int, 2 * l_g >(), l_prv, l_po, l_sr, true );
      store_one( std::integral_constant< int, 2 * l_g + 1 >(), l_prv, l_po, l_sr, true );
    } );
  };

  f32x16 l_acc0[2], l_acc1[2];
  l_acc0[0] = l_acc0[1] = l_acc1[0] = l_acc1[1] = f32x16( 0.0f );
  int32_t l_t = 0;
  for( ; l_t + 1 < l_np; l_t += 2 ) {
    panel( l_t, l_acc0, l_acc1 );
    panel( l_t + 1, l_acc1, l_acc0 );
  }
  if( l_t < l_np ) {
    panel( l_t, l_acc0, l_acc1 );
    last_stores( l_acc0 );
  }
  else {
    last_stores( l_acc1 );
  }
}

}  // namespace

int launch_contract_panel( ContractArgs const & a, hipStream_t stream ) {
  bool const l_res_a = a.M <= a.N;
  int32_t const l_S = l_res_a ? a.M : a.N;
  int32_t const l_L = l_res_a ? a.N : a.M;
  int32_t const l_sl = l_res_a ? a.sn_b : a.sm_a;
  // the kernel's own assumptions, checked before any launch
  if(    l_S < 1 || l_S > 256 || a.K < 1 || a.K > kPnKMax || a.C != 1 || l_sl < 0 || !a.out_off32
      || l_L < ( l_S > 128 ? 64 : 128 )
      || a.out_bytes == 0 || a.out_bytes > kPnOob || a.out_bf16 || a.first_touch != ETIR_KTYPE_ZERO
      || ( a.last_touch != ETIR_KTYPE_UNDEFINED && a.last_touch != ETIR_KTYPE_RELU ) || a.panel_grid < 1 ) {
    return fail( ETIR_COMPILATION_FAILED, "panel contraction: shape or touch kernels outside the kernel's range" );
  }
  int32_t const l_pl = ( l_S > 128 ) ? 64 : 128;
  int32_t const l_np = ( l_L + l_pl - 1 ) / l_pl;
  uint32_t const l_grid = (uint32_t) std::min( l_np, a.panel_grid );
  bool const l_relu = ( a.last_touch == ETIR_KTYPE_RELU );
  bool const l_lfast = ( l_sl == 1 );
  auto go = [&]( auto sp_c, auto ra_c, auto relu_c, auto lf_c ) {
    hipLaunchKernelGGL( ( contract_panel_kernel< decltype( sp_c )::value, decltype( ra_c )::value,
                                                 decltype( relu_c )::value, decltype( lf_c )::value > ),
                        dim3( l_grid ), dim3( kPnThreads ), 0, stream, a, l_np );
  };
  auto pick_lf = [&]( auto sp_c, auto ra_c, auto relu_c ) {
    if( l_lfast ) go( sp_c, ra_c, relu_c, std::true_type() );
    else          go( sp_c, ra_c, relu_c, std::false_type() );
  };
  auto pick_relu = [&]( auto sp_c, auto ra_c ) {
    if( l_relu ) pick_lf( sp_c, ra_c, std::true_type() );
    else         pick_lf( sp_c, ra_c, std::false_type() );
  };
  auto pick_side = [&]( auto sp_c ) {
    if( l_res_a ) pick_relu( sp_c, std::true_type() );
    else          pick_relu( sp_c, std::false_type() );
  };
  if( l_S > 128 ) pick_side( std::integral_constant< int, 256 >() );
  else            pick_side( std::integral_constant< int, 128 >() );
  return ETIR_SUCCESS;
}

}  // namespace etir
