// xq_fa_mma.hip — FLASH_ATTN_EXT decode / short multi-query verify on the
// gfx950 matrix cores: Q quantisation, the KV stream and the merge of the wave
// states happen in one kernel; with several KV splits the ascending-order split
// merge runs as fa_reduce right after it on the same stream (one memory round
// trip there costs less than the cross-XCD round trips a last-arriving
// workgroup needs to merge inside this kernel: 64.4 against 70.4 us per call
// on the 32k q8_0 decode, 21.4 against 28.8 us on the 4k f16 decode).
//
// Work decomposition. A workgroup owns one (sequence, KV head, query tile,
// KV split). A split is a contiguous row range, or (AUTO and LENGTH split
// modes) every n_splits-th group of NW slices. Its NW waves stream disjoint
// 16-row slices of the split (slice j goes to wave j % NW) through private
// double-buffered LDS rings filled by
// global_load_lds, each with its own online softmax and no workgroup barrier
// in the row loop. The wave states are merged through LDS at the end; with
// several splits each workgroup writes a partial state (unnormalised output,
// running maximum, running sum) for fa_reduce.
//
// Products (M x N x K of each MFMA):
//   scores  S = K Q^T, A = 16 KV rows, B = 16 (query, head) pairs.
//           q8_0 / q4_0 K: v_mfma_i32_16x16x32_i8 per 32-element block, the
//           exact integer block dot of ggml's vec_dot_q8_0_q8_0 /
//           vec_dot_q4_0_q8_0 between the K block and the q8_0-quantised Q
//           row, then scaled by d_k * d_q (one 4-block v_mfma_f32_16x16x1f32
//           forms the products of four blocks in the score layout) in f32.
//           q4_0 nibbles n enter as the signed bytes 16*(n - 8) against
//           d_q/16: the integer dot is 16x ggml's and the scale 1/16 of it,
//           both exact, so every product, and so every score, is ggml's.
//           F16 / E5M2 K: v_mfma_f32_16x16x32_f16 on the exact f16 K with Q
//           split into f16 hi + lo parts (the NATIVE policy uses hi alone).
//   values  O^T = V^T W^T, A = 16 head dims x the slice's rows, B = the
//           weights of 16 pairs. The score tile's output registers (lane =
//           pair, four consecutive rows) hold exactly the rows a lane gives
//           the B operand, so the softmax weights never leave registers and
//           every per-pair quantity (maximum, sum, rescale factor) is
//           lane-local.
//           q8_0 / q4_0 V: v_mfma_f32_16x16x16_f16 on the exact integer values
//           as f16 (q4_0's high nibbles as 16x theirs, undone exactly at the
//           merge), once against the high and once against the low parts of
//           w * 2^S_p * d_v as f16: each product formed in f32 by v_fma_mix, its f16
//           rounding h and the remainder w * 2^S_p * d_v - h as f16, about 22
//           significant bits (ggml multiplies the weight by the f32 dequantized
//           value, one f32 rounding). 2^S_p, a power of two per pair sized from
//           the block scales the pair has seen, keeps every high part in f16's
//           normal range whatever V's scale (a product w * d_v would fall into
//           subnormals, and then to zero, as V's magnitude shrinks); it enters
//           the weights' exponent argument and leaves at the merge, both
//           exactly.
//           F16 / E5M2 V: v_mfma_f32_16x16x16_f16 on the exact f16 V, once
//           against the weights' f16 high parts and once against their low
//           parts, about 22 significant bits of every weight (the weights lie
//           in (0, 16]). Two 16x16x16 products read the same V registers; one
//           16x16x32 product would need the rows repeated (two moves per tile).
// Online softmax in base 2 (scores pre-multiplied by log2 e) with a lazy
// maximum: the running maximum moves only when a slice exceeds it by more
// than 8, so accumulator rescales are rare; weights are taken relative to the
// maximum plus 4 and so stay in (0, 16].
//
// Rows a pair does not see (mask -inf, past its causal limit or the split)
// never touch its state, as ggml's loop skips them: a slice that holds such a
// row or a non-finite score runs "careful" — the scores of unseen rows become
// -inf whatever K holds, and the weight x scale products of quantized V's
// unseen rows are masked to +0 whatever their scale holds. Non-finite V
// reaches exactly the dims it sits in, of the pairs that see its row, as in
// ggml's per-dim accumulation: F16/E5M2 V elements that are Inf/NaN enter the
// shared V operand as 0 and are added to those accumulator elements after
// the products (every slice scans its V rows), and an Inf/NaN block scale's
// product keeps a zero low part. Range calls (positions) additionally turn a
// row whose output or normaliser is not finite into NaN in full (the split
// reducer's poisoning).
#include <type_traits>

#include "xq_fa_common.h"

namespace xq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr bool is_quant(int kt) { return kt == XQ_TYPE_Q8_0 || kt == XQ_TYPE_Q4_0; }

constexpr int kSub = 16;               // KV rows per wave slice
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kLazyMax = 8.0f;       // base-2 headroom before the running maximum moves
constexpr float kPOff = 4.0f;          // weights are exp2(x - max - 4), in (0, 16]

// Mask source of calls without a mask: one zero f16 pair.
__device__ uint32_t g_fa_zero_mask[1];

template <int KT, int D, int MT>
struct DecCfg {
    static constexpr int REC = rec_bytes(KT, D);
    static constexpr int SLICE = kSub * REC;
    static constexpr int CS = REC % 16 == 0 ? 16 : 4;  // bytes per lane per global_load_lds
    static constexpr int CPS = SLICE / CS;             // chunks per slice per tensor
    static constexpr int NIS = (CPS + 63) / 64;        // wave loads per slice per tensor
    static constexpr int NB = D / kQK;                 // 32-element blocks per row
    static constexpr int NPP = 16 * MT;
    static constexpr bool QUANT = is_quant(KT);
    static constexpr int QRB = QUANT ? D + 8 * NB : 0;      // LDS Q image row bytes (int8 path; d_q then 4*NB spare bytes that keep the stride)
    static constexpr int RING_W = 2 * 2 * SLICE;            // per wave: 2 stages x (K, V)
    static constexpr int MASK_W = 2 * MT * 512;             // per wave: 2 stages x MT x 2 f16 pairs per lane
    static constexpr int FIXED = NPP * QRB + 2 * 8 * NPP * 4 + 64;
    static constexpr bool NW8 = 8 * (RING_W + MASK_W) + FIXED <= 160 * 1024 && !(MT == 2 && D == 256);
    static constexpr int NW = NW8 ? 8 : 4;
    static constexpr int RING = NW * RING_W;
    static constexpr int QIMG = RING;                       // Q image after the K/V rings
    static constexpr int MASKR = QIMG + NPP * QRB;          // mask rings after the Q image
    static constexpr int MS = D + 4;                        // merge row stride (floats)
    static constexpr int MERGE = NW * 16 * MS * 4;
    static constexpr int LOOP = MASKR + NW * MASK_W;
    static constexpr int SMEM = LOOP > MERGE ? LOOP : MERGE;
    static constexpr bool FITS = SMEM + 2 * NW * NPP * 4 + 64 <= 160 * 1024;
};

// 8 K bytes of block b of a q8_0 / q4_0 record in LDS as an int8 MFMA
// operand: the block's elements in lane group g's eight k slots. q8_0: elements
// 8g..8g+7. q4_0 (elements 0..15 are the low nibbles of bytes 0..15, 16..31
// the high nibbles): the two nibbles of bytes 4g..4g+3, elements 4g..4g+3 then
// 16+4g..16+4g+3 (the Q operand takes the same order; the block's integer dot
// does not depend on it); nibble n becomes the signed byte 16*(n - 8) =
// (n << 4) ^ 0x80.
template <int KT>
XQ_DEV int64_t k_block_bytes(const uint8_t* rec, int b, int g) {
    constexpr int BB = KT == XQ_TYPE_Q8_0 ? 34 : 18;
    const int sh = (BB * b + 2) & 3;  // 0 or 2, depends on b only
    if constexpr (KT == XQ_TYPE_Q4_0) {
        const int off = BB * b + 2 + 4 * g;
        const uint32_t w = sh == 0 ? lds_u32(rec + off) : __builtin_amdgcn_alignbyte(lds_u32(rec + off + 2), lds_u32(rec + off - 2), 2);
        const uint32_t lo = ((w << 4) & 0xf0f0f0f0u) ^ 0x80808080u;
        const uint32_t hi = (w & 0xf0f0f0f0u) ^ 0x80808080u;
        return (int64_t)(((uint64_t)hi << 32) | lo);
    }
    const int off = BB * b + 2 + 8 * g;
    uint32_t w0, w1;
    if (sh == 0) {
        w0 = lds_u32(rec + off);
        w1 = lds_u32(rec + off + 4);
    } else {
        const uint32_t x = lds_u32(rec + off - 2), m = lds_u32(rec + off + 2), c = lds_u32(rec + off + 6);
        w0 = __builtin_amdgcn_alignbyte(m, x, 2);
        w1 = __builtin_amdgcn_alignbyte(c, m, 2);
    }
    return (int64_t)(((uint64_t)w1 << 32) | w0);
}

// V^T operands of one q8_0 block: the signed bytes 0 (tile 0) and 1 (tile 1)
// of the rows' 16-bit words x0..x3 as f16 pairs (rows 0,1 and rows 2,3),
// exact. Each pair is two SDWA conversions of sign-extended bytes, the second
// writing the high half and keeping the low one. The words are 16-bit asm
// operands: the conversions read their low bytes only, so the registers' high
// halves need no clearing after the LDS loads. The trailing s_nop gives the
// two wait states an MFMA reading a VGPR needs after a VALU wrote it (the
// compiler's hazard tracking does not see into the asm).
XQ_DEV void q8_vt_f16(uint16_t x0, uint16_t x1, uint16_t x2, uint16_t x3, uint32_t (&A0)[2], uint32_t (&A1)[2]) {
    asm("v_cvt_f16_i16_sdwa %0, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%6) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %1, sext(%7) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%4) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %2, sext(%5) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%6) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_1\n\t"
        "v_cvt_f16_i16_sdwa %3, sext(%7) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1\n\t"
        "s_nop 1"
        : "=&v"(A0[0]), "=&v"(A0[1]), "=&v"(A1[0]), "=&v"(A1[1])
        : "v"(x0), "v"(x1), "v"(x2), "v"(x3));
}

// Bytes b0, b1 (16-bit asm operands, high halves unread) as the 16-bit halves of
// one word, zero-extended: one v_perm and no clearing of the loads' high bits.
XQ_DEV uint32_t pack_bytes(uint16_t b0, uint16_t b1) {
    uint32_t r;
    asm("v_perm_b32 %0, %1, %2, %3" : "=v"(r) : "v"(b1), "v"(b0), "s"(0x0c040c00u));
    return r;
}

// B operand of a quantized-V value product: the f32 weights w0..w3 (rows 0..3)
// times the rows' f16 block scales as f16 high + low parts. Each product w*d
// is formed in f32 by v_fma_mix and rounded to f16 (the high part h); the low
// part is the remainder w*d - h, formed by one more v_fma_mix from the same
// operands with -h as the addend and rounded to f16, so h + l holds about 22
// significant bits of w*d (h is within 2^-11 of w*d). Packed as rows
// (0,1), (2,3) of the high parts, then of the low parts. The scale of row i is
// the low (HI = false) or high half of d[i]. s_nop as in q8_vt_f16.
template <bool HI>
XQ_DEV void wd_f16x2(float w0, float w1, float w2, float w3, uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                     uint32_t& b01, uint32_t& b23, uint32_t& l01, uint32_t& l23) {
    if constexpr (HI)
        asm("v_fma_mixlo_f16 %0, %4, %8, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixhi_f16 %0, %5, %9, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixlo_f16 %1, %6, %10, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixhi_f16 %1, %7, %11, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixlo_f16 %2, %4, %8, -%0 op_sel:[0,1,0] op_sel_hi:[0,1,1]\n\t"
            "v_fma_mixhi_f16 %2, %5, %9, -%0 op_sel:[0,1,1] op_sel_hi:[0,1,1]\n\t"
            "v_fma_mixlo_f16 %3, %6, %10, -%1 op_sel:[0,1,0] op_sel_hi:[0,1,1]\n\t"
            "v_fma_mixhi_f16 %3, %7, %11, -%1 op_sel:[0,1,1] op_sel_hi:[0,1,1]\n\t"
            "s_nop 1"
            : "=&v"(b01), "=&v"(b23), "=&v"(l01), "=&v"(l23)
            : "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(d0), "v"(d1), "v"(d2), "v"(d3));
    else
        asm("v_fma_mixlo_f16 %0, %4, %8, 0 op_sel:[0,0,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixhi_f16 %0, %5, %9, 0 op_sel:[0,0,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixlo_f16 %1, %6, %10, 0 op_sel:[0,0,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixhi_f16 %1, %7, %11, 0 op_sel:[0,0,0] op_sel_hi:[0,1,0]\n\t"
            "v_fma_mixlo_f16 %2, %4, %8, -%0 op_sel:[0,0,0] op_sel_hi:[0,1,1]\n\t"
            "v_fma_mixhi_f16 %2, %5, %9, -%0 op_sel:[0,0,1] op_sel_hi:[0,1,1]\n\t"
            "v_fma_mixlo_f16 %3, %6, %10, -%1 op_sel:[0,0,0] op_sel_hi:[0,1,1]\n\t"
            "v_fma_mixhi_f16 %3, %7, %11, -%1 op_sel:[0,0,1] op_sel_hi:[0,1,1]\n\t"
            "s_nop 1"
            : "=&v"(b01), "=&v"(b23), "=&v"(l01), "=&v"(l23)
            : "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(d0), "v"(d1), "v"(d2), "v"(d3));
}

// f16 exponent field of a block scale, 0 for Inf/NaN (those never size the
// value scaling: a row that holds one and is seen makes its pairs NaN anyway).
XQ_DEV int scale_exp(uint32_t h) {
    const int e = (int)((h >> 10) & 31u);
    return e == 31 ? 0 : e;
}

// Halves of w (a pair of f16) that are Inf or NaN (all-ones exponent) set to 0.
XQ_DEV uint32_t f16x2_zero_nonfinite(uint32_t w) {
    const uint32_t t = ((w & 0x7c007c00u) + 0x04000400u) & 0x80008000u;  // 0x8000 per non-finite half
    return w & ~((t >> 15) * 0xffffu);
}

// Nonzero when any f16 half of w is Inf or NaN.
XQ_DEV uint32_t f16x2_nonfinite(uint32_t w) { return ((w & 0x7c007c00u) + 0x04000400u) & 0x80008000u; }
// 0xffff in each f16 half of w that is finite, 0 in each Inf/NaN half.
XQ_DEV uint32_t f16x2_finite_mask(uint32_t w) { return ~((f16x2_nonfinite(w) >> 15) * 0xffffu); }
// Nonzero when any E5M2 byte of w is Inf or NaN.
XQ_DEV uint32_t e5m2x4_nonfinite(uint32_t w) { return ((w & 0x7c7c7c7cu) + 0x04040404u) & 0x80808080u; }

// The largest of four scores in two instructions (v_max3 then v_max; a quiet
// NaN operand is ignored, as fmaxf does, and the scores are never signalling
// NaNs, so the canonicalising moves the compiler adds around fmaxf are not
// needed).
XQ_DEV float max4(float a, float b, float c, float d) {
    float t, r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(t) : "v"(a), "v"(b), "v"(c));
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(t), "v"(d));
    return r;
}

// Reductions over the four 16-lane rows (lanes l, l^16, l^32, l^48) by
// permlane swaps; every lane gets the same bits ((r0 op r2) op (r1 op r3)).
XQ_DEV float xrow_max(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
XQ_DEV float xrow_sum(float x) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// HBM -> LDS without registers: lane l's CS bytes from base + off land at
// lds + l*CS (m0 = the LDS address of lane 0). Written as inline assembly so
// the compiler's wait insertion, which cannot tell the ring stages apart and
// would wait for every DMA in flight before any ring read, adds no waits: the
// kernel's explicit vmcnt waits order each DMA group before the reads of its
// stage, and the asm's memory clobber keeps LDS reads on their side of them.
// One wait state separates the m0 write from its use by the DMA. NT marks the
// load non-temporal: KV rows are read once (2 % faster on the 4k f16 decode).
// Only records that are whole 128-byte lines take it: a line shared by two
// heads' records (272-byte q8_0 records) is otherwise fetched once into L2 for
// both, and non-temporal loads fetch it twice (+11 % HBM traffic, no faster).
// The 32-pair verify tile keeps ordinary loads (1 % slower with them).
template <int CS, bool NT = false>
XQ_DEV void lds_dma(const uint8_t* base, uint32_t off, uint8_t* lds) {
    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    if constexpr (CS == 16 && NT)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
    else if constexpr (CS == 16)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
    else if constexpr (NT)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1 nt" ::"v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
    else
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(m0)
                     : "memory", "m0");
}

// Head dim held by accumulator register i of value tile (block c, half t) in
// lane group lg. q8_0 / F16 / E5M2 tiles take dims 32c + 2n + t (n = tile
// row), q4_0 tiles dims 32c + 16t + n (low / high nibbles of byte n).
template <int KT>
XQ_DEV int acc_dim(int c, int t, int lg, int i) {
    return KT == XQ_TYPE_Q4_0 ? 32 * c + 16 * t + 4 * lg + i : 32 * c + 8 * lg + 2 * i + t;
}

template <int KT, int D, int MT, bool SOFTCAP, bool HI_ONLY>
__global__ __launch_bounds__((64 * DecCfg<KT, D, MT>::NW)) void fa_dec(FaArgs a) {
    using C = DecCfg<KT, D, MT>;
    constexpr int REC = C::REC, SLICE = C::SLICE, CS = C::CS, CPS = C::CPS, NIS = C::NIS;
    constexpr int NB = C::NB, NPP = C::NPP, NW = C::NW, QRB = C::QRB;
    constexpr bool QUANT = C::QUANT;
    constexpr int BB = KT == XQ_TYPE_Q8_0 ? 34 : 18;
    constexpr int NT = 64 * NW;
    constexpr uint32_t kNegInfH2 = 0xfc00fc00u;  // f16 pair (-inf, -inf)

    __shared__ __attribute__((aligned(16))) uint8_t smem[C::SMEM];
    __shared__ float sM[NW][NPP], sL[NW][NPP];
    __shared__ int sProg[NW];  // slices each wave has finished (issue-priority balancing)

    const uint32_t n_wg = (uint32_t)a.n_splits * a.n_qtiles * a.Hkv * a.B;
    uint32_t wg = xcd_remap(blockIdx.x, n_wg);
    // logical order: query tile fastest, then KV head, split, sequence, so the
    // heads reading the same rows are neighbours on one XCD (shared L2)
    const int qt = wg % a.n_qtiles;
    wg /= a.n_qtiles;
    const int g_kv = wg % a.Hkv;
    wg /= a.Hkv;
    const int split = wg % a.n_splits;
    const int b = wg / a.n_splits;
    const int iq0 = qt * a.QT;
    const int nqt = min(a.QT, a.NQ - iq0);
    const int npa = nqt * a.G;
    const int wave = wave_id();
    const int lane = lane_id();
    const int tid = threadIdx.x;
    const int lr = lane & 15;
    const int lg = lane >> 4;

    // ---- rows of this split (row indices are 32-bit: the host keeps L below
    //      2^30): split_rows contiguous rows, or (interleave) every n_splits-th
    //      group of NW 16-row slices (one per wave) from group `split` on, so
    //      that the splits' row counts differ by at most one group whatever L
    //      is. With positions each pair sees rows below its causal limit
    const int r0 = a.interleave ? split * kSub * NW : split * (int)a.split_rows;
    int r_end = a.interleave ? (int)a.L : (int)min(a.L, (int64_t)r0 + a.split_rows);
    int r_all = r_end;  // rows below every pair's limit (per-row limits apply past it)
    if (a.positions) {
        int lmax = 0, lmin = (int)a.L;
        for (int qq = 0; qq < nqt; ++qq) {
            const int32_t pos = a.positions[iq0 + qq];
            const int lim = pos < a.origin ? 0 : (int)min(a.L, (int64_t)pos - a.origin + 1);
            lmax = max(lmax, lim);
            lmin = min(lmin, lim);
        }
        r_end = min(r_end, lmax);
        r_all = min(r_end, lmin);
    }
    const uint8_t* kb = a.k + (int64_t)(b / a.rk3) * a.k_nb3 + (int64_t)g_kv * a.k_nb2;
    const uint8_t* vb = a.v + (int64_t)(b / a.rv3) * a.v_nb3 + (int64_t)g_kv * a.v_nb2;

    // ---- per-wave ring [stage][K | V][SLICE]; chunk c = 64 i + lane of a
    //      slice is (row c / (REC/CS), byte (c % (REC/CS)) * CS)
    uint8_t* ring = smem + wave * C::RING_W;
    uint32_t ko[NIS], vo[NIS];
    int crow[NIS];
#pragma unroll
    for (int i = 0; i < NIS; ++i) {
        const int c = i * 64 + lane;
        crow[i] = c / (REC / CS);
        ko[i] = (uint32_t)(crow[i] * a.k_nb1 + (c % (REC / CS)) * CS);
        vo[i] = (uint32_t)(crow[i] * a.v_nb1 + (c % (REC / CS)) * CS);
    }
    // The ring is refilled in half-slice units: the K unit of a slice (NIS K
    // loads, then its 2*MT mask loads) and its V unit (NIS V loads), each
    // exactly that many vector-memory instructions. A unit reads constant
    // per-lane offsets from a wave-uniform row base; in the slice that holds the
    // last live row, the rows past it re-read that row.
    // (r_end >= 1 wherever a unit is issued.)
    auto unit = [&](const uint8_t* base, int64_t nb1, const uint32_t (&off)[NIS], int t0, uint8_t* dst) {
        if (t0 + kSub <= r_end) {
            const uint8_t* bt = base + (int64_t)t0 * nb1;
#pragma unroll
            for (int i = 0; i < NIS; ++i)
                if (CPS % 64 == 0 || i + 1 < NIS || lane < CPS % 64) lds_dma<CS, MT == 1 && REC % 128 == 0>(bt, off[i], dst + i * 64 * CS);
        } else {
            // rows from tr = min(t0, r_end - 1); lane rows clamp to r_end - 1, so
            // every offset is non-negative and below 16 rows (the whole slice
            // may lie past the end). The lane's row relative to tr is formed
            // from its fixed slice row and two wave-uniform terms, so no
            // per-lane row index is carried through the loop for this branch.
            const int tr = min(t0, r_end - 1);
            const int d0 = t0 - tr, last = r_end - 1 - tr;
            const uint8_t* bt = base + (int64_t)tr * nb1;
#pragma unroll
            for (int i = 0; i < NIS; ++i) {
                const int rel = min(crow[i] + d0, last);  // row - tr
                const uint32_t o = off[i] + (uint32_t)(rel - crow[i]) * (uint32_t)nb1;
                if (CPS % 64 == 0 || i + 1 < NIS || lane < CPS % 64) lds_dma<CS, MT == 1 && REC % 128 == 0>(bt, o, dst + i * 64 * CS);
            }
        }
    };

    // ---- per-pair state of this lane's pairs 16m + lr (identical in the four lane groups)
    float m_run[MT], l_run[MT], slope2[MT];
    int lim[MT];
    uint32_t moff[MT];  // mask: the lane's offset in the sequence's plane (row, head, element 4lg)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        m_run[m] = -INFINITY;
        l_run[m] = 0.0f;
        slope2[m] = kLog2e;
        lim[m] = r_end;  // padding pairs (zero Q, never stored) run like valid ones
        const int p = 16 * m + lr;
        const bool ok = p < npa;
        const int qq = ok ? p / a.G : 0, h = g_kv * a.G + (ok ? p % a.G : 0);
        if (ok) {
            if (a.positions) {
                const int32_t pos = a.positions[iq0 + qq];
                lim[m] = pos < a.origin ? 0 : (int)min((int64_t)r_end, (int64_t)pos - a.origin + 1);
            }
            slope2[m] = alibi_slope(a, h) * kLog2e;
        }
        // padding pairs read the first pair's mask row (always valid memory); with
        // no mask every pair reads the first f16 pair of a zero row
        moff[m] = a.mask ? (uint32_t)((int64_t)(iq0 + qq) * a.m_nb1 + (int64_t)(h % a.m_ne2) * a.m_nb2) + 8u * lg : 0u;
    }
    // mask of a slice: lane (lr, lg) brings rows t + 4lg + 2k, +1 (k = 0, 1) of its
    // pair's mask row as one f16 pair into its slot of the wave's mask ring, in the
    // same DMA group as K and V, so the loop holds no register-destination loads.
    // Rows at or past the mask's end read the row's first pair (they lie past every
    // pair's limit and are replaced by -inf); the pair at the last row, when L is
    // odd, reads the aligned dword that holds it (the host requires 4-byte aligned
    // mask rows).
    // The address is the sequence's mask plane (wave-uniform, in SGPRs; the
    // slice's first row joins it) plus the lane's 32-bit offset moff[m] (its
    // pair's row and head, then element 4lg; the host keeps a plane below 2^31
    // bytes), so a full slice's mask loads take no vector instructions.
    const int mcols = a.mask ? (int)a.L : 0;
    uint8_t* mring = smem + C::MASKR + wave * C::MASK_W;
    const uint8_t* mplane = a.mask ? a.mask + (int64_t)(b % a.m_ne3) * a.m_nb3 : (const uint8_t*)g_fa_zero_mask;
    auto load_mask = [&](int t, int st) {
        if (!a.mask) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int k = 0; k < 2; ++k) lds_dma<4>(mplane, 0u, mring + (st * MT + m) * 512 + k * 256);
        } else if (t + kSub <= mcols) {
            const uint8_t* mt = mplane + 2 * (int64_t)t;
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int k = 0; k < 2; ++k) lds_dma<4>(mt, moff[m] + 4u * k, mring + (st * MT + m) * 512 + k * 256);
        } else {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int r = t + 4 * lg + 2 * k;
                    const uint32_t o = r < mcols ? moff[m] + (uint32_t)(2 * t + 4 * k) : moff[m] - 8u * lg;
                    lds_dma<4>(mplane, o, mring + (st * MT + m) * 512 + k * 256);
                }
        }
    };

    const int step = a.interleave ? kSub * NW * a.n_splits : kSub * NW;
    int t0 = r0 + kSub * wave;
    constexpr int VD = D / 64;
    constexpr int PPW = (NPP + NW - 1) / NW;
    // Units: K_j, mask_j, V_j, then the same for slice j+1 (the loop keeps this
    // issue order).
    auto k_unit = [&](int tt, int st) {
        unit(kb, a.k_nb1, ko, tt, ring + st * 2 * SLICE);
        load_mask(tt, st);
    };
    auto v_unit = [&](int tt, int st) { unit(vb, a.v_nb1, vo, tt, ring + st * 2 * SLICE + SLICE); };

    // ---- int8 path: wave w quantizes pairs w, w + NW, ... (VD floats per lane)
    //      into the Q image in LDS (pairs >= npa are zero). The Q rows come by
    //      DMA into the wave's ring stage 1, ahead of stage 0's units, and are
    //      waited for alone (loads complete in order), so Q does not wait behind
    //      the ring; stage 1's units follow once the rows are read.
    //      Float K: the f16 hi / lo B operands straight from Q, then the units.
    constexpr bool QSTAGE = QUANT && PPW * D * 4 <= 2 * SLICE;
    uint8_t* sQ = smem + C::QIMG;
    h8 qh[QUANT ? 1 : MT][QUANT ? 1 : NB], ql[QUANT ? 1 : MT][QUANT ? 1 : NB];
    if constexpr (QUANT) {
        constexpr int LPB = kQK / VD;
        float x[PPW][VD];
        if constexpr (QSTAGE) {
            uint8_t* qst = ring + 2 * SLICE;
#pragma unroll
            for (int k = 0; k < PPW; ++k) {
                const int p = wave + k * NW;  // wave-uniform
                if (p < npa) {
                    const int qq = p / a.G, h = g_kv * a.G + p % a.G;
                    const uint8_t* row = a.q + (int64_t)b * a.q_nb3 + (int64_t)(iq0 + qq) * a.q_nb1 + (int64_t)h * a.q_nb2;
#pragma unroll
                    for (int i = 0; i < VD; ++i) lds_dma<4>(row, (uint32_t)(64 * i + lane) * 4u, qst + (k * D + 64 * i) * 4);
                }
            }
            if (t0 < r_end) {
                k_unit(t0, 0);
                v_unit(t0, 0);
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NIS + 2 * MT) : "memory");  // Q rows landed
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int k = 0; k < PPW; ++k) {
                const bool ok = wave + k * NW < npa;
#pragma unroll
                for (int j = 0; j < VD; ++j) x[k][j] = ok ? ((const float*)qst)[k * D + lane * VD + j] : 0.0f;
            }
        } else {
#pragma unroll
            for (int k = 0; k < PPW; ++k) {
                const int p = wave + k * NW;
                const bool ok = p < npa;
                const float* src = (const float*)a.q;
                if (ok) {
                    const int qq = p / a.G, h = g_kv * a.G + p % a.G;
                    src = (const float*)(a.q + (int64_t)b * a.q_nb3 + (int64_t)(iq0 + qq) * a.q_nb1 + (int64_t)h * a.q_nb2);
                }
#pragma unroll
                for (int j = 0; j < VD; ++j) x[k][j] = ok ? src[lane * VD + j] : 0.0f;
            }
            if (t0 < r_end) {
                k_unit(t0, 0);
                v_unit(t0, 0);
            }
        }
#pragma unroll
        for (int k = 0; k < PPW; ++k) {
            const int p = wave + k * NW;
            if (p >= NPP) break;
            uint8_t* img = sQ + p * QRB;
            // ggml-cpu x86 quantize_row_q8_0: d = amax/127 (stored as f16),
            // id = 127/amax, q = round-half-even(x * id)
            float amax = 0.0f;
#pragma unroll
            for (int j = 0; j < VD; ++j) amax = fmaxf(amax, fabsf(x[k][j]));
            amax = fmaxf(amax, dpp<0xB1>(amax));
            amax = fmaxf(amax, dpp<0x4E>(amax));
            amax = fmaxf(amax, dpp<0x141>(amax));
            if constexpr (LPB == 16) amax = fmaxf(amax, dpp<0x140>(amax));
            const float dblk = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < VD; ++j) {
                const int qv = (int)rintf(x[k][j] * id);
                packed |= (uint32_t)(uint8_t)(int8_t)qv << (8 * j);
            }
            if constexpr (VD == 4)
                *(uint32_t*)(img + 4 * lane) = packed;
            else
                *(uint16_t*)(img + 2 * lane) = (uint16_t)packed;
            if ((lane % LPB) == 0) {
                const int blk = (lane * VD) / kQK;
                const float dqv = f16_bits_to_f32(f32_to_f16_bits(dblk));
                // q4_0 K bytes are 16x the signed nibbles: d_q / 16 (exact) keeps each
                // product d_k * d_q * dot
                ((float*)(img + D))[blk] = KT == XQ_TYPE_Q4_0 ? dqv * 0.0625f : dqv;
            }
        }
        if (t0 + step < r_end) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // staged Q rows read
            k_unit(t0 + step, 1);
            v_unit(t0 + step, 1);
        }
    } else {
        // ring stage 0 first: its loads overlap the Q loads' round trip
        if (t0 < r_end) {
            k_unit(t0, 0);
            v_unit(t0, 0);
        }
        // The pair's f32 Q elements, every load issued before any is used (a
        // padding pair reads pair 0's row, always valid, and is zeroed at use):
        // one round trip in all, overlapping stage 0's
        float xq[MT][NB][8];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int p = 16 * m + lr;
            const int pp = p < npa ? p : 0;
            const int qq = pp / a.G, h = g_kv * a.G + pp % a.G;
            const float* src = (const float*)(a.q + (int64_t)b * a.q_nb3 + (int64_t)(iq0 + qq) * a.q_nb1 + (int64_t)h * a.q_nb2);
#pragma unroll
            for (int c = 0; c < NB; ++c)
#pragma unroll
                for (int j = 0; j < 8; ++j) xq[m][c][j] = src[32 * c + 8 * lg + j];
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const bool ok = 16 * m + lr < npa;
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                // Q = f16 hi + f16 lo (lo = 0 for the NATIVE policy); NaN as ggml's f16 conversion
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float xv = ok ? xq[m][c][j] : 0.0f;
                    const uint32_t hb = f32_to_f16_bits(xv);
                    qh[m][c][j] = __builtin_bit_cast(_Float16, (uint16_t)hb);
                    ql[m][c][j] = HI_ONLY ? (_Float16)0.0f
                                            : __builtin_bit_cast(_Float16, (uint16_t)f32_to_f16_bits(xv - f16_bits_to_f32(hb)));
                }
            }
        }
        if (t0 + step < r_end) {
            k_unit(t0 + step, 1);
            v_unit(t0 + step, 1);
        }
    }
    __syncthreads();

    // ---- B operands of the score product: pair 16m + lr, elements 8lg..8lg+7 of each block
    int64_t qb[QUANT ? MT : 1][QUANT ? NB : 1];
    // dqb[m][q]: d_q of block 4q + lg of the lane's pair (the B operand of the
    // 4-block scale product)
    float dqb[QUANT ? MT : 1][QUANT ? NB / 4 : 1];
    if constexpr (QUANT) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const uint8_t* img = sQ + (16 * m + lr) * QRB;
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                // q4_0: elements 4lg..4lg+3 and 16+4lg..16+4lg+3, K's order
                qb[m][c] = KT == XQ_TYPE_Q4_0
                               ? (int64_t)(((uint64_t)lds_u32(img + 32 * c + 16 + 4 * lg) << 32) | lds_u32(img + 32 * c + 4 * lg))
                               : *(const int64_t*)(img + 32 * c + 8 * lg);
                // without softcap the score scale (times log2 e) rides on d_q: the
                // block products then give the base-2 scores directly
                if (c % 4 == 0) dqb[m][c / 4] = ((const float*)(img + D))[c + lg] * (SOFTCAP ? 1.0f : a.scale * kLog2e);
            }
        }
    }
    const float sc2 = a.scale * kLog2e;
    const float cap2 = a.softcap * kLog2e;

    f4 acc[MT][2 * NB];
    // the f16 pair (1024, 1024) in a VGPR, opaque to constant folding: each
    // q4_0 value operand half then takes one v_and_or (a VOP3 cannot hold it
    // as a literal)
    uint32_t k6400 = 0;
    if constexpr (KT == XQ_TYPE_Q4_0) asm("v_mov_b32 %0, 0x64006400" : "=v"(k6400));
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < 2 * NB; ++n) acc[m][n] = f4{0.0f, 0.0f, 0.0f, 0.0f};

    // ---- scores s[m][i] of the slice in ring stage ST: row 4lg + i, pair 16m + lr
    auto scores = [&](auto st_tag, float (&s)[MT][4]) {
        constexpr int ST = decltype(st_tag)::value;
        const uint8_t* Ks = ring + ST * 2 * SLICE;
        if constexpr (QUANT) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[m][i] = 0.0f;
            // blocks in batches of four: the K operand reads, the 4-block f32 product
            // dks[m][4j + i] = d_k(row 4lg + i, block c0 + j) * d_q(pair, block c0 + j)
            // (exact: two f16 significands), the independent integer block dots,
            // then s += dks * float(block dot) as ggml's vec_dot_q8_0_q8_0 /
            // vec_dot_q4_0_q8_0 accumulate (d = d_k*d_q, then sum += d * sumi)
#pragma unroll
            for (int c0 = 0; c0 < NB; c0 += 4) {
                int64_t ka[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) ka[j] = k_block_bytes<KT>(Ks + lr * REC, c0 + j, lg);
                // A operand of the scale product: lane (lr, lg) gives d_k of row lr, block c0 + lg
                const float dkl = (float)*(const _Float16*)(Ks + lr * REC + BB * (c0 + lg));
                f16v dks[MT];
#pragma unroll
                for (int m = 0; m < MT; ++m)
                    dks[m] = __builtin_amdgcn_mfma_f32_16x16x1f32(dkl, dqb[m][c0 / 4], f16v{}, 0, 0, 0);
                i4 I[MT][4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        I[m][j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(ka[j], qb[m][c0 + j], i4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int m = 0; m < MT; ++m)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            s[m][i] = fmaf((float)I[m][j][i], dks[m][4 * j + i], s[m][i]);
                        }
            }
        } else {
            f4 sc[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) sc[m] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                h8 kf;
                if constexpr (KT == XQ_TYPE_F16) {
                    kf = *(const h8*)(Ks + lr * REC + 64 * c + 16 * lg);
                } else {  // E5M2: byte b -> f16 bits b << 8
                    const uint2 w = *(const uint2*)(Ks + lr * REC + 32 * c + 8 * lg);
                    const uint4 hv = {__builtin_amdgcn_perm(w.x, w.x, 0x010c000cu), __builtin_amdgcn_perm(w.x, w.x, 0x030c020cu),
                                      __builtin_amdgcn_perm(w.y, w.y, 0x010c000cu), __builtin_amdgcn_perm(w.y, w.y, 0x030c020cu)};
                    kf = __builtin_bit_cast(h8, hv);
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    sc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qh[m][c], sc[m], 0, 0, 0);
                    if (!HI_ONLY) sc[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, ql[m][c], sc[m], 0, 0, 0);
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) s[m][i] = sc[m][i];
        }
    };

    // ---- values of the slice in ring stage ST, block c:
    //      acc[m][2c + t] += V^T(rows 4lg..4lg+3, tile dims) x W^T, as two
    //      products: the weights' high parts, then their low parts
    //      pw: f32 weights (row 4lg + i, pair 16m + lr; quantized V: times
    //      2^S_p); seenm: careful slice's masks of the rows the pair sees;
    //      Bf: F16/E5M2 weight operands; vsan: F16/E5M2: Inf/NaN V elements
    //      enter the shared operand as 0; q8_0/q4_0: an Inf/NaN scale's product
    //      keeps a zero low part
    auto values = [&](auto st_tag, int c, const float (&pw)[MT][4], auto careful_tag, const uint32_t (&seenm)[MT][2],
                      const h8 (&Bf)[MT], bool vsan) {
        constexpr int ST = decltype(st_tag)::value;
        constexpr bool careful = decltype(careful_tag)::value;  // a separate copy: no mask selects when false
        const uint8_t* Vs = ring + ST * 2 * SLICE + SLICE;
        uint32_t X[4];
        uint16_t X16[4];  // q8_0: the rows' 16-bit words (16-bit asm operands)
        if constexpr (KT == XQ_TYPE_Q4_0) {
            // byte lr of rows (0,1) and (2,3) as the halves of X[0], X[1]
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint8_t* vr = Vs + (4 * lg + 2 * e) * REC + 18 * c + 2 + lr;
                X[e] = pack_bytes(vr[0], vr[REC]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint8_t* vr = Vs + (4 * lg + e) * REC;
                if constexpr (KT == XQ_TYPE_Q8_0)
                    X16[e] = *(const uint16_t*)(vr + 34 * c + 2 + 2 * lr);
                else if constexpr (KT == XQ_TYPE_F16)
                    X[e] = lds_u32(vr + 2 * (32 * c + 2 * lr));
                else
                    X[e] = lds_u16(vr + 32 * c + 2 * lr);
            }
        }
        if constexpr (QUANT) {
            // B: w * 2^S * d_v as f16 high parts (Bh) and low parts (Bl) of rows
            // (0,1), (2,3); the pair's power of two 2^S keeps every high part in
            // f16's normal range
            uint32_t dvw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) dvw[i] = lds_u32(Vs + (4 * lg + i) * REC + ((BB * c) & ~3));
            const bool dhi = ((BB * c) & 2) != 0;  // the scale sits in the high half of its dword
            h4 Bh[MT], Bl[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                uint32_t b01, b23, l01, l23;
                if (dhi)
                    wd_f16x2<true>(pw[m][0], pw[m][1], pw[m][2], pw[m][3], dvw[0], dvw[1], dvw[2], dvw[3], b01, b23, l01, l23);
                else
                    wd_f16x2<false>(pw[m][0], pw[m][1], pw[m][2], pw[m][3], dvw[0], dvw[1], dvw[2], dvw[3], b01, b23, l01, l23);
                if constexpr (careful) {
                    if (vsan) {
                        // an Inf/NaN scale: the low part of its product (Inf - Inf)
                        // is set to 0, so the high part alone gives q * d's Inf / NaN
                        l01 &= f16x2_finite_mask(b01);
                        l23 &= f16x2_finite_mask(b23);
                    }
                    // rows the pair does not see add 0, whatever their scale holds
                    b01 &= seenm[m][0];
                    b23 &= seenm[m][1];
                    l01 &= seenm[m][0];
                    l23 &= seenm[m][1];
                }
                Bh[m] = __builtin_bit_cast(h4, uint2{b01, b23});
                Bl[m] = __builtin_bit_cast(h4, uint2{l01, l23});
            }
            // A: the integer values of tile t's dims in rows (0,1), (2,3) as f16 (exact)
            uint32_t A0[2], A1[2];
            if constexpr (KT == XQ_TYPE_Q8_0) {
                q8_vt_f16(X16[0], X16[1], X16[2], X16[3], A0, A1);
            } else {
                // q4_0: the low nibble n (dim lr of the block) as 1024 + n - 1032 =
                // n - 8, the high nibble (dim 16 + lr) unshifted as 1024 + 16n - 1152
                // = 16(n - 8); both exact. Tile 1's accumulators hold 16x their
                // values (every rounding scales with them) until the merge.
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const uint32_t w = X[e];
                    const uint32_t lo = (w & 0x000f000fu) | k6400;
                    const uint32_t hi = (w & 0x00f000f0u) | k6400;
                    A0[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, lo) + h2{(_Float16)-1032.0f, (_Float16)-1032.0f});
                    A1[e] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, hi) + h2{(_Float16)-1152.0f, (_Float16)-1152.0f});
                }
            }
            // the four rows against the high parts, then against the low parts: two
            // 16x16x16 products read the same V registers (one 16x16x32 product
            // would need the rows repeated in four registers, two moves per tile)
            const h4 At0 = __builtin_bit_cast(h4, uint2{A0[0], A0[1]});
            const h4 At1 = __builtin_bit_cast(h4, uint2{A1[0], A1[1]});
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                acc[m][2 * c] = __builtin_amdgcn_mfma_f32_16x16x16f16(At0, Bh[m], acc[m][2 * c], 0, 0, 0);
                acc[m][2 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(At1, Bh[m], acc[m][2 * c + 1], 0, 0, 0);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                acc[m][2 * c] = __builtin_amdgcn_mfma_f32_16x16x16f16(At0, Bl[m], acc[m][2 * c], 0, 0, 0);
                acc[m][2 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(At1, Bl[m], acc[m][2 * c + 1], 0, 0, 0);
            }
        } else {
            // A: f16 pairs of rows (0,1), (2,3) of tiles t = 0, 1 (exact)
            uint32_t A0[2], A1[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint32_t x0 = X[2 * e], x1 = X[2 * e + 1];
                if constexpr (KT == XQ_TYPE_F16) {
                    A0[e] = __builtin_amdgcn_perm(x1, x0, 0x05040100u);
                    A1[e] = __builtin_amdgcn_perm(x1, x0, 0x07060302u);
                } else {  // E5M2: byte b -> f16 bits b << 8
                    A0[e] = __builtin_amdgcn_perm(x1, x0, 0x040c000cu);
                    A1[e] = __builtin_amdgcn_perm(x1, x0, 0x050c010cu);
                }
                if (vsan) {
                    A0[e] = f16x2_zero_nonfinite(A0[e]);
                    A1[e] = f16x2_zero_nonfinite(A1[e]);
                }
            }
            const h4 At0 = __builtin_bit_cast(h4, uint2{A0[0], A0[1]});
            const h4 At1 = __builtin_bit_cast(h4, uint2{A1[0], A1[1]});
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const h4 bh = __builtin_shufflevector(Bf[m], Bf[m], 0, 1, 2, 3);
                acc[m][2 * c] = __builtin_amdgcn_mfma_f32_16x16x16f16(At0, bh, acc[m][2 * c], 0, 0, 0);
                acc[m][2 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(At1, bh, acc[m][2 * c + 1], 0, 0, 0);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const h4 bl = __builtin_shufflevector(Bf[m], Bf[m], 4, 5, 6, 7);
                acc[m][2 * c] = __builtin_amdgcn_mfma_f32_16x16x16f16(At0, bl, acc[m][2 * c], 0, 0, 0);
                acc[m][2 * c + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(At1, bl, acc[m][2 * c + 1], 0, 0, 0);
            }
        }
    };

    // ---- one 16-row slice j from ring stage S (S static: the loop is unrolled by
    //      two). The K unit of slice j+2 is issued once this slice's K and mask
    //      reads are done, its V unit once the V reads are done, so three units
    //      are in flight while a slice computes.
    // Waves w and w + 4 share a SIMD, whose issue arbiter favours the older
    // wave: left alone, waves 4..7 finish their rows ~25 % later and then run
    // without a partner while the workgroup waits for them. Each wave posts its
    // progress and takes issue priority while it is behind its partner (ties go
    // to the younger wave).
    // quantized V: pair p's accumulators hold sum w * 2^S_p * d_v * q and its
    // weight sum sum w * 2^S_p (the weights are formed as exp2(x - mu + S_p)), with
    // S_p = 25 - the largest block-scale exponent field among the rows p has
    // seen so far (so w * 2^S_p * |d_v| < 2^15). S_p depends on p's rows only,
    // so a pair's bits do not depend on the pairs that share its tile; it only
    // falls, and every fall rescales p's accumulator column and sum by a power of two.
    int e_max[MT], s_exp[MT];
    int e_min = -1;  // wave-uniform: the smallest e_max over the pairs (-1 while one has seen no row)
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        e_max[m] = -1;
        s_exp[m] = 0;
    }
    int done = 0;
    if (lane == 0) sProg[wave] = 0;
    auto balance = [&]() {
        if constexpr (NW == 8) {
            const int other = __hip_atomic_load(&sProg[wave ^ 4], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (done < other || (done == other && wave >= 4))
                __builtin_amdgcn_s_setprio(1);
            else
                __builtin_amdgcn_s_setprio(0);
        }
    };
    auto slice = [&](int t, auto stage_tag) {
        constexpr int S = decltype(stage_tag)::value;
        const bool n1 = t + step < r_end, n2 = t + 2 * step < r_end;  // slices j+1, j+2 exist
        balance();
        // K_j and mask_j are complete once only the later units are outstanding:
        // V_j, then (when slice j+1 exists) K_j+1 + mask_j+1 and V_j+1; loads
        // complete in order
        if (n1)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * NIS + 2 * MT) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NIS) : "memory");
        __builtin_amdgcn_wave_barrier();
        float s[MT][4];
        scores(stage_tag, s);

        // -- the mask pairs of this slice, then the K unit (and mask) of slice j+2
        //    into the stage this slice's K and mask used
        uint32_t mw[MT][2];
        const uint8_t* ms = mring + S * MT * 512 + 4 * lane;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            mw[m][0] = lds_u32(ms + m * 512);
            mw[m][1] = lds_u32(ms + m * 512 + 256);
        }
        if (n2) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // K and mask reads of this stage done
            k_unit(t + 2 * step, S);
        }

        // -- V_j complete: later units K_j+1 + mask, V_j+1, K_j+2 + mask
        if (n2)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * NIS + 4 * MT) : "memory");
        else if (n1)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NIS + 2 * MT) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __builtin_amdgcn_wave_barrier();
        // -- F16/E5M2 V: a non-finite element must reach exactly its own dim of
        //    the pairs that see its row, as ggml's per-dim accumulation does
        //    (VKQ += v * vs). It must not reach the pairs that do not see the
        //    row through the shared V operand, and Inf times a weight's low
        //    part could give NaN where the product is Inf. Lane (lr, lg) scans
        //    its sixteenth of rows 4lg..4lg+3 here (0 * x is +-0 for finite x,
        //    NaN otherwise), the reads overlapping the softmax; when any element
        //    is Inf/NaN the V operands are sanitised and the bad elements are
        //    added after the products (vrb: bit i = row 4lg + i holds one)
        uint32_t vrb = 0;
        if constexpr (!QUANT) {
            constexpr int ES = KT == XQ_TYPE_F16 ? 2 : 1;
            constexpr int SPAN = ES * D / 16;  // bytes per lane per row (8..32)
            const uint8_t* Vs = ring + S * 2 * SLICE + SLICE;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint8_t* vr = Vs + (4 * lg + i) * REC + lr * SPAN;
                uint32_t bad = 0;
                if constexpr (KT == XQ_TYPE_F16) {
                    h2 z = h2{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
                    for (int k = 0; k < SPAN / 16; ++k) {
                        const uint4 w = *(const uint4*)(vr + 16 * k);
                        const h2 zero = h2{(_Float16)0.0f, (_Float16)0.0f};
                        z = __builtin_elementwise_fma(__builtin_bit_cast(h2, w.x), zero, z);
                        z = __builtin_elementwise_fma(__builtin_bit_cast(h2, w.y), zero, z);
                        z = __builtin_elementwise_fma(__builtin_bit_cast(h2, w.z), zero, z);
                        z = __builtin_elementwise_fma(__builtin_bit_cast(h2, w.w), zero, z);
                    }
                    bad = __builtin_bit_cast(uint32_t, z) & 0x7fff7fffu;
                } else {
#pragma unroll
                    for (int k = 0; k < SPAN / 8; ++k) {
                        const uint2 w = *(const uint2*)(vr + 8 * k);
                        bad |= e5m2x4_nonfinite(w.x) | e5m2x4_nonfinite(w.y);
                    }
                }
                vrb |= bad ? 1u << i : 0u;
            }
        }
        // quantized V: lane l reads the block scales of row l/4 (largest exponent
        // field er), used after the softmax
        // (dsan: some block scale of the slice is Inf/NaN)
        int er = 0;
        bool dsan = false;
        if constexpr (QUANT) {
            const uint8_t* vr = ring + S * 2 * SLICE + SLICE + (lane >> 2) * REC;
            uint32_t hs;
            if constexpr (NB == 8) {
                const int b0 = 2 * (lane & 3);
                hs = lds_u16(vr + BB * b0) | (lds_u16(vr + BB * (b0 + 1)) << 16);
                er = max(scale_exp(hs & 0xffffu), scale_exp(hs >> 16));
            } else {
                hs = lds_u16(vr + BB * (lane & 3));
                er = scale_exp(hs);
            }
            dsan = __builtin_amdgcn_ballot_w64(f16x2_nonfinite(hs) != 0) != 0;
        }
        // -- online softmax (base 2)
        float x[MT][4];
        bool nonfin = false;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const h2 mh = __builtin_bit_cast(h2, mw[m][i >> 1]);
                const float v = SOFTCAP ? cap2 * tanhf(s[m][i] * a.scale) : QUANT ? s[m][i] : s[m][i] * sc2;
                x[m][i] = fmaf(slope2[m], (float)mh[i & 1], v);
            }
            // a sum of finite scores (|x| far below the f32 range) is finite
            // exactly when every score is: one test for -inf, +inf and NaN
            nonfin |= !__builtin_isfinite((x[m][0] + x[m][1]) + (x[m][2] + x[m][3]));
        }
        // careful slice: rows past a pair's limit, masked rows, non-finite
        // scores or (quantized V) a non-finite block scale; unseen rows (past
        // the limit, mask -inf) become -inf
        const bool careful = t + kSub > r_all || __builtin_amdgcn_ballot_w64(nonfin) != 0 || dsan;
        if (careful) {
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const h2 mh = __builtin_bit_cast(h2, mw[m][i >> 1]);
                    const bool seen = t + 4 * lg + i < lim[m] && (float)mh[i & 1] != -INFINITY;
                    x[m][i] = seen ? x[m][i] : -INFINITY;
                }
        }
        // A pair's maximum moves only when one of its lanes holds a score above
        // the bound, so the lanes' own maxima are tested first and the
        // cross-lane reductions run only for a slice where one does (in the
        // first slices, and rarely after): the same maxima either way
        float lmax[MT];
        bool over = false;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            lmax[m] = max4(x[m][0], x[m][1], x[m][2], x[m][3]);
            over |= lmax[m] > m_run[m] + kLazyMax;
        }
        if (__builtin_amdgcn_ballot_w64(over)) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const float mt = xrow_max(lmax[m]);
                // integer maxima: every rescale factor is an exact power of two and
                // the pair's power 2^S_p folds exactly into the exponent argument
                const float mnew = mt > m_run[m] + kLazyMax ? ceilf(mt) : m_run[m];
                const float al = mnew == m_run[m] ? 1.0f : __builtin_amdgcn_exp2f(m_run[m] - mnew);
                l_run[m] *= al;
#pragma unroll
                for (int n = 0; n < 2 * NB; ++n) acc[m][n] *= al;
                m_run[m] = mnew;
            }
        }
        // -- quantized V: each pair's largest block-scale exponent over the rows
        //    of this slice it sees; lane l reads blocks of row l/4, a quad holds
        //    its row's maximum, every lane gathers its lane group's four rows
        uint32_t seenmask[MT][2];  // careful slice: f16-half masks of the rows the pair sees
        if constexpr (QUANT) {
            // fast test: no row's scale exceeds every pair's bound, so no pair's
            // S moves (the exact per-pair update below runs only otherwise)
            if (__builtin_amdgcn_ballot_w64(er > e_min)) {
                er = max(er, dpp_i<0xB1>(er));
                er = max(er, dpp_i<0x4E>(er));  // quad q holds row q's largest exponent
                int ep[MT];
                if (!careful) {
                    // every pair sees every row: the slice's maximum, wave-wide
                    int e = max(er, dpp_i<0x141>(er));
                    e = max(e, dpp_i<0x140>(e));
                    auto r = __builtin_amdgcn_permlane32_swap((uint32_t)e, (uint32_t)e, false, false);
                    e = max((int)r[0], (int)r[1]);
                    auto q = __builtin_amdgcn_permlane16_swap((uint32_t)e, (uint32_t)e, false, false);
                    e = __builtin_amdgcn_readfirstlane(max((int)q[0], (int)q[1]));
#pragma unroll
                    for (int m = 0; m < MT; ++m) ep[m] = e;
                } else {
                    // the rows the pair sees: gather the lane group's four rows
                    int erow[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) erow[i] = __shfl(er, (lane & ~15) + 4 * i);
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        int e = -1;
#pragma unroll
                        for (int i = 0; i < 4; ++i) e = max(e, x[m][i] != -INFINITY ? erow[i] : -1);
                        auto r = __builtin_amdgcn_permlane32_swap((uint32_t)e, (uint32_t)e, false, false);
                        e = max((int)r[0], (int)r[1]);
                        auto q = __builtin_amdgcn_permlane16_swap((uint32_t)e, (uint32_t)e, false, false);
                        ep[m] = max((int)q[0], (int)q[1]);
                    }
                }
                int emn = 1 << 30;
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const bool grow = ep[m] > e_max[m];
                    if (__builtin_amdgcn_ballot_w64(grow)) {
                        const int s_new = grow ? 25 - max(ep[m], 1) : s_exp[m];
                        const float f = __builtin_ldexpf(1.0f, s_new - s_exp[m]);  // exact power of two
#pragma unroll
                        for (int n = 0; n < 2 * NB; ++n) acc[m][n] *= f;
                        l_run[m] *= f;
                        s_exp[m] = s_new;
                        e_max[m] = grow ? ep[m] : e_max[m];
                    }
                    emn = min(emn, e_max[m]);
                }
                emn = min(emn, dpp_i<0xB1>(emn));
                emn = min(emn, dpp_i<0x4E>(emn));
                emn = min(emn, dpp_i<0x141>(emn));
                emn = min(emn, dpp_i<0x140>(emn));
                {
                    auto r = __builtin_amdgcn_permlane32_swap((uint32_t)emn, (uint32_t)emn, false, false);
                    emn = min((int)r[0], (int)r[1]);
                    auto q = __builtin_amdgcn_permlane16_swap((uint32_t)emn, (uint32_t)emn, false, false);
                    e_min = __builtin_amdgcn_readfirstlane(min((int)q[0], (int)q[1]));
                }
            }
            if (careful) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    seenmask[m][0] = (x[m][0] != -INFINITY ? 0xffffu : 0u) | (x[m][1] != -INFINITY ? 0xffff0000u : 0u);
                    seenmask[m][1] = (x[m][2] != -INFINITY ? 0xffffu : 0u) | (x[m][3] != -INFINITY ? 0xffff0000u : 0u);
                }
            }
        }
        float pw[MT][4];
        h8 Bf[MT];  // F16/E5M2 V: weights as f16 high parts (products 0..3), low parts (4..7)
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            // quantized V: weights times 2^S_p (exact: integer maximum, integer S_p)
            const float mu = (m_run[m] == -INFINITY ? 0.0f : m_run[m] + kPOff) - (QUANT ? (float)s_exp[m] : 0.0f);
#pragma unroll
            for (int i = 0; i < 4; ++i) pw[m][i] = __builtin_amdgcn_exp2f(x[m][i] - mu);
            l_run[m] += (pw[m][0] + pw[m][1]) + (pw[m][2] + pw[m][3]);
            if constexpr (!QUANT) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    Bf[m][i] = (_Float16)pw[m][i];
                    Bf[m][4 + i] = (_Float16)(pw[m][i] - (float)Bf[m][i]);
                }
            }
        }
        // -- F16/E5M2 V: whether a row of the slice holds an Inf/NaN element (the
        //    scan above), and which
        bool vsan = false;
        uint32_t rowbad = 0;  // rows of the slice holding a non-finite V element (vsan only)
        if constexpr (!QUANT) {
            vsan = __builtin_amdgcn_ballot_w64(vrb != 0) != 0;
            if (vsan) {
                uint32_t rb = vrb;
                rb |= (uint32_t)dpp_i<0xB1>((int)rb);
                rb |= (uint32_t)dpp_i<0x4E>((int)rb);
                rb |= (uint32_t)dpp_i<0x141>((int)rb);
                rb |= (uint32_t)dpp_i<0x140>((int)rb);  // every lane of the row group: the flags of its four rows
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) rowbad |= (uint32_t)__builtin_amdgcn_readlane((int)rb, 16 * g4) << (4 * g4);
            }
        }
        if constexpr (QUANT) {
            if (careful) {
#pragma unroll
                for (int c = 0; c < NB; ++c) values(stage_tag, c, pw, std::true_type{}, seenmask, Bf, dsan);
            } else {
#pragma unroll
                for (int c = 0; c < NB; ++c) values(stage_tag, c, pw, std::false_type{}, seenmask, Bf, dsan);
            }
        } else {
#pragma unroll
            for (int c = 0; c < NB; ++c) values(stage_tag, c, pw, std::false_type{}, seenmask, Bf, vsan);
            if (vsan) {
                // the bad elements of each bad row j: pair 16m + lr adds w * v to
                // its accumulator element of that dim when it sees row j (its
                // weight comes from lane (lr, j/4), register j % 4); the lane
                // holds dims 32c + 8lg + 2i + t in acc[m][2c + t][i]
                float ws[MT][4];
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int i = 0; i < 4; ++i) ws[m][i] = x[m][i] != -INFINITY ? pw[m][i] : -1.0f;
                const uint8_t* Vs = ring + S * 2 * SLICE + SLICE;
                for (int j = 0; j < kSub; ++j) {
                    if (!((rowbad >> j) & 1u)) continue;
                    const int src = lr + 16 * (j >> 2), ji = j & 3;
                    float wj[MT];
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const float sel = ji == 0 ? ws[m][0] : ji == 1 ? ws[m][1] : ji == 2 ? ws[m][2] : ws[m][3];
                        wj[m] = __shfl(sel, src);
                    }
                    const uint8_t* vr = Vs + j * REC;
#pragma unroll
                    for (int c = 0; c < NB; ++c) {
                        float v[8];
                        if constexpr (KT == XQ_TYPE_F16) {
                            const h8 hv = *(const h8*)(vr + 2 * (32 * c + 8 * lg));
#pragma unroll
                            for (int e = 0; e < 8; ++e) v[e] = (float)hv[e];
                        } else {
                            const uint2 w = *(const uint2*)(vr + 32 * c + 8 * lg);
#pragma unroll
                            for (int e = 0; e < 8; ++e)
                                v[e] = f16_bits_to_f32((((e < 4 ? w.x : w.y) >> (8 * (e & 3))) & 0xffu) << 8);
                        }
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            if (__builtin_isfinite(v[e])) continue;
#pragma unroll
                            for (int m = 0; m < MT; ++m)
                                if (wj[m] >= 0.0f) acc[m][2 * c + (e & 1)][e >> 1] += wj[m] * v[e];
                        }
                    }
                }
            }
        }

        // -- the V unit of slice j+2 into the stage this slice's V used
        if (n2) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // V reads of this stage done
            v_unit(t + 2 * step, S);
        }
        ++done;
        if (NW == 8 && lane == 0) __hip_atomic_store(&sProg[wave], done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    };
    for (; t0 < r_end; t0 += 2 * step) {
        slice(t0, std::integral_constant<int, 0>{});
        if (t0 + step < r_end) slice(t0 + step, std::integral_constant<int, 1>{});
    }
    __builtin_amdgcn_s_setprio(0);
    if (NW == 8 && lane == 0) __hip_atomic_store(&sProg[wave], 1 << 30, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);  // done: never behind

    // ---- merge the wave states per 16-pair group through LDS (fixed wave order)
    const int64_t rows_per_seq = (int64_t)a.NQ * a.H;
    // [NW][16][MS]: rows padded by 4 floats so the 16 rows a write instruction
    // touches start on different banks (unpadded, a 16-way conflict). With one
    // pair group whose 16 rows fit in a wave's own ring (OWN), each wave writes
    // them there as soon as its rows are done, without waiting for the others:
    // its ring is its own, and no other wave reads it.
    constexpr int MS = C::MS;
    constexpr bool OWN = MT == 1 && 16 * MS * 4 <= C::RING_W;
    constexpr int WST = OWN ? C::RING_W / 4 : 16 * MS;  // a wave's rows (floats)
    if constexpr (!OWN) __syncthreads();  // every wave is done with its ring and the Q image
    float* mb = (float*)smem;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        // quantized V: l and the accumulators hold 2^S_p times their values (exact)
        const float unscale = __builtin_ldexpf(1.0f, -s_exp[m]);
        const float lt = xrow_sum(QUANT ? l_run[m] * unscale : l_run[m]);
        if (lg == 0) {
            sM[wave][16 * m + lr] = m_run[m] == -INFINITY ? -INFINITY : m_run[m] + kPOff;
            sL[wave][16 * m + lr] = lt;
        }
        float* mw = mb + wave * WST + lr * MS;
        // the lane's dims of block c as 16-byte writes (acc_dim's layout);
        // padding pairs are never read
        if (16 * m + lr < npa) {
#pragma unroll
            for (int c = 0; c < NB; ++c) {
                const f4 x0 = QUANT ? acc[m][2 * c] * unscale : acc[m][2 * c];
                // q4_0 tile 1: 16x its values (exact power of two)
                const f4 x1 = QUANT ? acc[m][2 * c + 1] * (KT == XQ_TYPE_Q4_0 ? unscale * 0.0625f : unscale) : acc[m][2 * c + 1];
                if constexpr (KT == XQ_TYPE_Q4_0) {
                    *(f4*)(mw + acc_dim<KT>(c, 0, lg, 0)) = x0;
                    *(f4*)(mw + acc_dim<KT>(c, 1, lg, 0)) = x1;
                } else {
                    *(f4*)(mw + acc_dim<KT>(c, 0, lg, 0)) = f4{x0[0], x1[0], x0[1], x1[1]};
                    *(f4*)(mw + acc_dim<KT>(c, 0, lg, 2)) = f4{x0[2], x1[2], x0[3], x1[3]};
                }
            }
        }
        __syncthreads();
        for (int e = tid; e < 16 * (D / 4); e += NT) {
            const int pl = e / (D / 4), d4 = e % (D / 4);
            const int p = 16 * m + pl;
            if (p >= npa) continue;
            float M = -INFINITY;
#pragma unroll
            for (int w = 0; w < NW; ++w) M = fmaxf(M, sM[w][p]);
            float Ls = 0.0f;
            f4 o = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int w = 0; w < NW; ++w) {
                const float mw_ = sM[w][p];
                const float ew = mw_ == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw_ - M);
                Ls = fmaf(sL[w][p], ew, Ls);
                o += ew * *(const f4*)(mb + w * WST + pl * MS + 4 * d4);
            }
            const int qq = p / a.G, h = g_kv * a.G + p % a.G, iq = iq0 + qq;
            const int64_t row = (int64_t)b * rows_per_seq + (int64_t)iq * a.H + h;
            const float Mn = M == -INFINITY ? -INFINITY : M * kLn2;  // natural-log units
            if (a.n_splits == 1) {
                float a1, inv, lse;
                fa_finalize(Ls == 0.0f ? -INFINITY : Mn, Ls, a.sinks != nullptr, a.sinks ? a.sinks[h] : 0.0f, a1, inv, lse);
                float* od = (float*)(a.dst + (int64_t)b * a.d_nb3 + (int64_t)iq * a.d_nb2 + (int64_t)h * a.d_nb1);
                f4 ov = (o * a1) * inv;
                if (a.poison) {
                    // the split reducer's rule with one split: a non-finite or
                    // negative sum, factor, normaliser or output poisons the row.
                    // A row's D/4 threads are one wave (D 256) or half of one (D 128).
                    const bool bad = !__builtin_isfinite(Ls) || Ls < 0.0f || !__builtin_isfinite(inv) ||
                                     (Ls != 0.0f && !__builtin_isfinite(lse)) || !__builtin_isfinite(ov[0]) ||
                                     !__builtin_isfinite(ov[1]) || !__builtin_isfinite(ov[2]) || !__builtin_isfinite(ov[3]);
                    const uint64_t rowmask = D == 256 ? ~0ull : (lane < 32 ? 0xffffffffull : 0xffffffff00000000ull);
                    if (__builtin_amdgcn_ballot_w64(bad) & rowmask) {
                        ov = f4{NAN, NAN, NAN, NAN};
                        lse = NAN;
                    }
                }
                *(f4*)(od + 4 * d4) = ov;
                if (d4 == 0 && a.lse) a.lse[row] = lse;
            } else {
                *(f4*)(a.part_o + (row * a.n_splits + split) * D + 4 * d4) = o;
                if (d4 == 0) a.part_ml[row * a.n_splits + split] = make_float2(Mn, Ls);
            }
        }
        if (m + 1 < MT) __syncthreads();  // the next group reuses the rows
    }
}

// ---------------------------------------------------------------- dispatch

using DecFn = void (*)(FaArgs);

// Variant of (type, head dim, pair tiles) for the call's softcap and Q policy
// (hi-only f16 Q exists for float K only).
template <int KT, int D, int MT>
static DecFn dec_inst(bool softcap, bool hi_only) {
    if constexpr (DecCfg<KT, D, MT>::FITS) {
        if constexpr (is_quant(KT)) {
            return softcap ? fa_dec<KT, D, MT, true, false> : fa_dec<KT, D, MT, false, false>;
        } else {
            if (softcap) return hi_only ? fa_dec<KT, D, MT, true, true> : fa_dec<KT, D, MT, true, false>;
            return hi_only ? fa_dec<KT, D, MT, false, true> : fa_dec<KT, D, MT, false, false>;
        }
    } else {
        return nullptr;
    }
}

template <int KT, int D>
static DecFn dec_for(int mt, bool softcap, bool hi_only) {
    return mt == 1 ? dec_inst<KT, D, 1>(softcap, hi_only) : mt == 2 ? dec_inst<KT, D, 2>(softcap, hi_only) : nullptr;
}

template <int KT, int D>
static int waves_for(int mt) {
    return mt == 1 ? DecCfg<KT, D, 1>::NW : DecCfg<KT, D, 2>::NW;
}

static DecFn dec_lookup(int kt, int d, int mt, int* waves, bool softcap = false, bool hi_only = false) {
#define XQ_DEC_CASE(T, DD) \
    case T: *waves = waves_for<T, DD>(mt); return dec_for<T, DD>(mt, softcap, hi_only);
    if (d == 128) {
        switch (kt) {
            XQ_DEC_CASE(XQ_TYPE_Q8_0, 128)
            XQ_DEC_CASE(XQ_TYPE_Q4_0, 128)
            XQ_DEC_CASE(XQ_TYPE_F16, 128)
            XQ_DEC_CASE(XQ_TYPE_E5M2, 128)
        }
    } else if (d == 256) {
        switch (kt) {
            XQ_DEC_CASE(XQ_TYPE_Q8_0, 256)
            XQ_DEC_CASE(XQ_TYPE_Q4_0, 256)
            XQ_DEC_CASE(XQ_TYPE_F16, 256)
            XQ_DEC_CASE(XQ_TYPE_E5M2, 256)
        }
    }
#undef XQ_DEC_CASE
    return nullptr;
}

bool fa_mma_available(int kt, int d, int qk_mode, int n_pairs) {
    if (n_pairs < 1 || n_pairs > 32) return false;
    if (is_quant(kt) && qk_mode != kQkInt8) return false;  // f32-Q scores on quantized K stay on VALU
    int w = 0;
    return dec_lookup(kt, d, (n_pairs + 15) / 16, &w) != nullptr;
}

int fa_mma_waves(int kt, int d, int n_pairs) {
    int w = 4;
    if (!dec_lookup(kt, d, (n_pairs + 15) / 16, &w)) return 0;
    return w;
}

// The mask rows are read as 4-byte pairs: every row base must be 4-byte aligned.
bool fa_mma_mask_ok(const FaArgs& a) {
    return !a.mask || ((uintptr_t)a.mask % 4 == 0 && a.m_nb1 % 4 == 0 && a.m_nb2 % 4 == 0 && a.m_nb3 % 4 == 0);
}

hipError_t fa_mma_launch(FaArgs a, const FaLaunch& L, hipStream_t stream) {
    const int D = (int)L.q->ne[0];
    const int kt = L.k->type;
    const int mt = (a.QT * a.G + 15) / 16;
    if (a.L >= (int64_t)1 << 30) return hipErrorInvalidValue;  // 32-bit row indices
    a.hi_only = is_quant(kt) ? 0 : (L.q_round_f16 ? 1 : 0);
    int waves = 0;
    DecFn fn = dec_lookup(kt, D, mt, &waves, a.softcap != 0.0f, a.hi_only != 0);
    if (!fn) return hipErrorInvalidValue;
    a.q = (const uint8_t*)L.q->data;
    a.q_nb1 = (int64_t)L.q->nb[1];
    a.q_nb2 = (int64_t)L.q->nb[2];
    a.q_nb3 = (int64_t)L.q->nb[3];
    if (!fa_mma_mask_ok(a)) return hipErrorInvalidValue;
    // the mask loads address a sequence's plane with 32-bit lane offsets
    if (a.mask && (int64_t)(a.NQ - 1) * a.m_nb1 + (int64_t)(a.m_ne2 - 1) * a.m_nb2 + 2 * a.L + 4 >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;
    const uint32_t n_wg = (uint32_t)a.n_splits * a.n_qtiles * a.Hkv * a.B;
    launch("fa_dec", fn, dim3(n_wg), dim3(64 * waves), stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.n_splits == 1) return e;
    return fa_reduce_launch(a, D, stream);
}

}  // namespace xq
