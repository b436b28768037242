// MXFP8 block-scaled GEMM for gfx950 with fused epilogues.
//
//   C[m, n] = epilogue( sum_k A[m, k] * 2^(sa[m, k/32]-127) * W[n, k] * 2^(sw[n, k/32]-127) )
//
// A (activations) is [M, K] e4m3fn with e8m0 scales [M, K/32]; W is the weight stored transposed,
// [N, K] e4m3fn with scales [N, K/32] -- both K-contiguous, the MX layout the adaLN kernel emits.
// The inner product runs on v_mfma_scale_f32_32x32x64_f8f6f4, which applies the e8m0 block scales
// in hardware, accumulating in fp32.
//
// Orientation: the MFMA's A operand is W (rows = output features n) and its B operand is A (columns
// = tokens m), so the accumulator of each lane holds four consecutive n of one token m per register
// group. Bias, GELU, bf16 rounding and the per-32 MX re-quantization along n are then lane-local
// (one exchange with lane ^ 32 completes a 32-wide block), and stores are 8-byte (bf16) or 4-byte
// (e4m3) vectors.
//
// Tiling: 256 (n) x 256 (m) x 128 (k) per workgroup of 4 waves, each wave a 128 x 128 block of
// 4 x 4 MFMA tiles (256 fp32 accumulators per lane). Operand codes are staged through LDS by
// direct-to-LDS buffer loads (buffer_load_dwordx4 ... lds, no VGPR round trip), with a
// 16-byte-chunk XOR swizzle so the MFMA operand reads of consecutive rows land on distinct banks.
// Each stage's loads are issued two stages ahead (the weight halves on a ring of five half-stage
// slots, the activations in two stage slots, so that a quarter of the loads can go out in the first
// half of a stage); operands are read per 64-deep slice into ping-pong registers, interleaved with
// the MFMAs of the other slice, and a stage needs one barrier. Block scales travel four stages at a
// time (16 bytes per row in one load, double-buffered): a row's scale bytes are 4 bytes per stage,
// so per-stage loads would cost an address-unit pass over 64 scattered rows for every 4 bytes.
//
// Measured on MI355X, these choices matter: direct-to-LDS loads with a non-zero scalar offset run
// ~45% slower than with the whole offset in the VGPR, so the offsets are VGPR sums of a per-lane part
// held through the k loop and a wave-uniform part; the loads are issued from inline asm, invisible
// to the compiler's wait-count pass, which would otherwise put a full vmcnt(0) before every LDS read
// and serialize the pipeline; and the k loop's order of reads, loads and MFMAs is pinned with
// scheduling barriers (10% faster than the compiler's own order, which moved MFMAs across the
// stage barriers and left the reads of a slice exposed).
//
// The kernel is persistent: one workgroup per CU walks tiles v = blockIdx.x, + gridDim.x, ... in an
// order where each XCD (workgroup ids are dealt round-robin over 8 XCDs) owns a contiguous,
// L2-friendly run of tiles grouped 4 deep along m (measured against 2, 8 and 16: 1-5% faster). The
// next tile's first stage is loaded while the current tile's epilogue runs, so the epilogue overlaps
// the next tile's load latency.
//
// Reference semantics: the ROW_MX projection epilogues of _qkv_cte_mx_impl / _dequant_row_mx
// (vllm_omni_neuron/kernels/nkilib/core/qkv/qkv_cte.py:3711-3750, 3996-4021) and of the MLP
// (kernels/nkilib/core/mlp/mlp_cte/mx/mlp_cte_mx_projection.py:630-668, GELU-tanh then
// quantize_mx in mlp_cte_mx_quantization.py:113-154); the torch statement is _mlp_ref_standard
// (kernels/nkilib/core/mlp/mlp_torch.py:401-599).
#include "wanmi_common.h"

#include <algorithm>

namespace wanmi {

constexpr int TN = 256;  // weight rows (output features) per tile
constexpr int TM = 256;  // tokens per tile
constexpr int BK = 128;  // k bytes per stage (4 MX blocks)
constexpr int kStageBytes = TN * BK + TM * BK;  // e4m3 codes of one stage (W rows, then A rows)
constexpr int kScaleGroup = 4;                    // stages per scale load (16 bytes per row)
constexpr int kVecFloats = 4 * 256;  // per tile: bias[n], col_scale[n], gate[n], row_scale[m]
constexpr int kGroupM = 4;  // m tiles per group (4: the XCD's 32 concurrent tiles are 4 m x 8 n)
constexpr int kCodeLoads = 16;   // direct-to-LDS loads per wave per stage of codes (16 x 1 KiB)

struct GemmArgs {
  const uint8_t* a;         // [M, lda]
  const uint8_t* a_scales;  // [M, K/32]
  const uint8_t* w;         // [N, K]
  const uint8_t* w_scales;  // [N, K/32]
  const float* row_scale;   // [M] or null
  const float* col_scale;   // [N] or null
  const float* bias;        // [N] or null
  const uint16_t* residual; // [M, ldo] bf16 (gated residual epilogue)
  const float* gate;        // [N]
  void* out;                // [M, ldo]
  uint8_t* out_scales;      // [M, N/32]
  float* row_sumsq;         // [M, N/128]: sum of squares of the bf16 outputs per 128-column block, or null
  int64_t sumsq_cols;       // blocks of columns [0, sumsq_cols) are summed
  int64_t sumsq_ld;         // row stride of row_sumsq in floats
  uint16_t* vt;             // V^T epilogue: [N/128][128][vt_ld] bf16
  int64_t vt_ld;
  int64_t M, N, K, lda, ldo;
  int tiles_m, tiles_n;
};

// gelu_tanh(x) = 0.5 x (1 + tanh(u)) = x / (1 + exp(-2u)),  u = sqrt(2/pi) (x + 0.044715 x^3);
// exp(-2u) = 2^(x (k0 + k1 x^2)) with k0 = -2 log2(e) sqrt(2/pi), k1 = 0.044715 k0 folded into one
// polynomial; hardware exp2 and reciprocal (relative error ~1e-7, far below the bf16 rounding that
// follows). Saturates correctly: exp(-2u) -> inf gives -0/+0, exp(-2u) -> 0 gives x.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float e = __builtin_amdgcn_exp2f(x * (-2.302208198144325f + -0.1029432395800235f * (x * x)));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// LDS byte offset of 16-byte chunk `chunk` of operand row `row`. The chunk index is XORed with
// f(row) = (row & 7) ^ ((row >> 3) & 1): the 16 lanes that one LDS cycle serves read rows r..r+15
// (64 banks of 4 bytes = two 128-byte rows), and f gives the eight even rows, and the eight odd
// rows, eight distinct chunk slots, so the MFMA operand reads are free of bank conflicts.
__device__ __forceinline__ int swz_f(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int swz(int row, int chunk) { return row * BK + ((chunk ^ swz_f(row)) << 4); }

// MFMA operands of one 64-deep k slice of a wave's 128 x 128 block: 4 weight-row and 4 token-row
// fragments (32 bytes per lane each) and their e8m0 scale bytes.
struct SliceOperands {
  i32x8 w[4];
  i32x8 a[4];
  int ws[4];
  int as[4];
};

// Per-lane offset of a lane's scale bytes in a scale buffer: row (lane & 31) of its 32-row fragment,
// 16 bytes per row, plus h = lane >> 5 (the lane's 32-block of the slice). Computed once per tile and
// held through the k loop, so a slice's scale reads cost no address arithmetic.
__device__ __forceinline__ uint32_t scale_lane_offset() {
  const uint32_t l = (uint32_t)fresh_lane_id();
  return (l & 31) * 16 + (l >> 5);
}

// Reads fragments [I0, I1) of slice s (0 or 1): weight rows i * 32 + r32 of the wave's 128-row half
// (wbase) and token rows wm * 128 + i * 32 + r32 (abase). Lane data: bytes 0-15 = k[64s + 16h, +16),
// bytes 16-31 = k[64s + 32 + 16h, +16); the lane's scale byte is block 2s + h of its row, byte
// 4q + 2s + h (q = the stage's position in its scale group) of the row's 16 scale bytes in `sc`
// ([2][256] x 16 B: W rows, then A rows), read as a byte so the MFMA takes it as is. The swizzle
// repeats every 16 rows, so a half read at its own base matches the whole stage read at row 128 wn.
template <int I0 = 0, int I1 = 4>
__device__ __forceinline__ void read_slice_r(const uint8_t* wbase, const uint8_t* abase, const uint32_t* sc, int q,
                                             int s, SliceOperands& op, int wn, int wm, int h, int r32, uint32_t sl) {
  const int c0 = s * 4 + h, c1 = s * 4 + 2 + h;
  const uint8_t* scb = reinterpret_cast<const uint8_t*>(sc) + 4 * q + 2 * s;
  const uint8_t* scw = scb + wn * 128 * 16 + sl;
  const uint8_t* sca = scb + (TN + wm * 128) * 16 + sl;
#pragma unroll
  for (int i = I0; i < I1; ++i) {
    const int rw = i * 32 + r32;
    const uint4 x0 = *reinterpret_cast<const uint4*>(wbase + swz(rw, c0));
    const uint4 x1 = *reinterpret_cast<const uint4*>(wbase + swz(rw, c1));
    op.w[i] = i32x8{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
    const int ra = wm * 128 + i * 32 + r32;
    const uint4 y0 = *reinterpret_cast<const uint4*>(abase + swz(ra, c0));
    const uint4 y1 = *reinterpret_cast<const uint4*>(abase + swz(ra, c1));
    op.a[i] = i32x8{(int)y0.x, (int)y0.y, (int)y0.z, (int)y0.w, (int)y1.x, (int)y1.y, (int)y1.z, (int)y1.w};
    op.ws[i] = (int)scw[i * 32 * 16];
    op.as[i] = (int)sca[i * 32 * 16];
  }
}

// The same from one stage buffer (weight rows, then token rows).
template <int I0 = 0, int I1 = 4>
__device__ __forceinline__ void read_slice(const uint8_t* base, const uint32_t* sc, int q, int s, SliceOperands& op,
                                           int wn, int wm, int h, int r32, uint32_t sl) {
  read_slice_r<I0, I1>(base + wn * 128 * BK, base + TN * BK, sc, q, s, op, wn, wm, h, r32, sl);
}

// One MFMA of weight fragment i against token fragment j. kSwap puts the tokens in the A operand,
// so the accumulator is transposed: lane l holds feature 32 i + (l & 31) and tokens
// 32 j + 8 g + 4 (l >> 5) + q (the V^T epilogue's layout); otherwise features along the registers.
template <bool kSwap>
__device__ __forceinline__ f32x16 mfma_tile(const i32x8& w, const i32x8& a, const f32x16& c, int ws, int as) {
  if constexpr (kSwap)
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, w, c, 0, 0, 0, as, 0, ws);
  else
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, a, c, 0, 0, 0, ws, 0, as);
}

// MFMAs of weight-row fragments [I0, I1) against all four token fragments.
template <int I0, int I1, bool kSwap = false>
__device__ __forceinline__ void mfma_rows(const SliceOperands& op, f32x16 (&acc)[4][4]) {
#pragma unroll
  for (int i = I0; i < I1; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = mfma_tile<kSwap>(op.w[i], op.a[j], acc[i][j], op.ws[i], op.as[j]);
}

// Per-tile buffer resources of one wave's direct-to-LDS loads.
struct TileLoads {
  u32x4 w, a, ws, as;
  int64_t m0, n0, m_valid;
};

__device__ __forceinline__ void tile_coords(const GemmArgs& g, int v, int64_t& m0, int64_t& n0) {
  const int total = g.tiles_m * g.tiles_n;
  int pid = v;
  if ((total & 7) == 0) pid = (v & 7) * (total >> 3) + (v >> 3);
  const int in_group = kGroupM * g.tiles_n;
  const int group = pid / in_group;
  const int first_m = group * kGroupM;
  const int gsz = min(g.tiles_m - first_m, kGroupM);
  const int tm = first_m + (pid % in_group) % gsz;
  const int tn = (pid % in_group) / gsz;
  n0 = (int64_t)tn * TN;
  m0 = (int64_t)tm * TM;
}

__device__ __forceinline__ TileLoads tile_loads(const GemmArgs& g, int v) {
  TileLoads t;
  tile_coords(g, v, t.m0, t.n0);
  const int64_t KB = g.K / 32;
  t.m_valid = min((int64_t)TM, g.M - t.m0);
  // Token rows past M fall outside the activation resources' extent and read as zero.
  t.w = buffer_rsrc(g.w + t.n0 * g.K, (uint32_t)(TN * g.K));
  t.a = buffer_rsrc(g.a + t.m0 * g.lda, (uint32_t)(t.m_valid * g.lda));
  t.ws = buffer_rsrc(g.w_scales + t.n0 * KB, (uint32_t)(TN * KB));
  t.as = buffer_rsrc(g.a_scales + t.m0 * KB, (uint32_t)(t.m_valid * KB));
  return t;
}

// !valid: an empty extent turns every load into a zero fill that moves no memory (branch-free)
__device__ __forceinline__ u32x4 maybe_empty(u32x4 r, bool valid) {
  r[2] = valid ? r[2] : 0u;
  return r;
}

// Direct-to-LDS loads of the codes of one stage into an LDS stage buffer. Wave w fills rows
// 64w .. 64w+63 of each operand tile, 8 rows (1 KiB) per instruction: in row group p (rows
// 64w + 8p + (l >> 3)) lane l lands in physical 16-byte slot l & 7 and fetches the logical chunk
// (l & 7) ^ f(row) = (l & 7) ^ (l >> 3) ^ (p & 1). The loads go in pairs (row group p of W and of
// the activations). A lane's offset splits into a per-lane part, row l >> 3 times the row stride
// plus its chunk (one value for even and one for odd row groups), and a wave-uniform part, the row
// group and the stage; the k loop holds the per-lane parts in registers (DmaLanes, computed once per
// tile), so a load costs one add. 24-bit multiplies suffice: rows < 256, and K and lda stay below
// 2^23 (checked on the host). Token rows past M fall outside the activations' descriptor extent and
// read as zero.
struct DmaLanes {
  uint32_t we, wo, ae, ao;  // W / activations, even / odd row groups
};

__device__ __forceinline__ DmaLanes dma_lanes(const GemmArgs& g) {
  const uint32_t l = (uint32_t)fresh_lane_id();
  const uint32_t srow = l >> 3;
  const uint32_t ce = ((l & 7) ^ srow) << 4, co = ce ^ 16u;
  const uint32_t rw = (uint32_t)__umul24(srow, (uint32_t)g.K), ra = (uint32_t)__umul24(srow, (uint32_t)g.lda);
  return DmaLanes{rw + ce, rw + co, ra + ce, ra + co};
}

// Row group p of both operands of stage kt into a stage buffer (weights, then activations; the
// simple loop's layout).
__device__ __forceinline__ void code_dma_pair(const GemmArgs& g, const TileLoads& t, const DmaLanes& dl, int kt,
                                              uint8_t* buf, int wave, int p, bool valid = true) {
  const uint32_t rg = (uint32_t)(wave * 64 + p * 8);  // first row of the row group
  const uint32_t kofs = (uint32_t)kt * BK;
  const uint32_t lds = lds_addr(buf) + rg * BK;
  const uint32_t sw = rg * (uint32_t)g.K + kofs, sa = rg * (uint32_t)g.lda + kofs;
  lds_dma_b128(maybe_empty(t.w, valid), ((p & 1) ? dl.wo : dl.we) + sw, lds);
  lds_dma_b128(maybe_empty(t.a, valid), ((p & 1) ? dl.ao : dl.ae) + sa, lds + TN * BK);
}

__device__ __forceinline__ void issue_codes(const GemmArgs& g, const TileLoads& t, int kt, uint8_t* buf, int wave,
                                            bool valid = true) {
  const DmaLanes dl = dma_lanes(g);
#pragma unroll
  for (int p = 0; p < 8; ++p) code_dma_pair(g, t, dl, kt, buf, wave, p, valid);
}

// Scale bytes of stage group grp (stages 4 grp .. 4 grp + 3, k-blocks [16 grp, 16 grp + 16)) ->
// `sc` ([2][256] x 16 B). Lane l of wave w copies the 16 bytes of row 64w + l of each operand.
__device__ __forceinline__ void issue_scales(const GemmArgs& g, const TileLoads& t, int grp, uint32_t* sc, int wave,
                                             bool valid = true) {
  const uint32_t KB = (uint32_t)(g.K / 32);
  const uint32_t v = (uint32_t)(wave * 64 + fresh_lane_id()) * KB + (uint32_t)grp * 16;
  const uint32_t ls = lds_addr(sc) + wave * 64 * 16;
  lds_dma_b128(maybe_empty(t.ws, valid), v, ls);
  lds_dma_b128(maybe_empty(t.as, valid), v, ls + TN * 16);
}

// The tile's epilogue vectors -> LDS (floats [0,256) bias, [256,512) col_scale, [512,768) gate,
// [768,1024) row_scale). Absent vectors are not loaded: their LDS slots keep the neutral values
// written once by init_vectors.
__device__ __forceinline__ void issue_vectors(const GemmArgs& g, const TileLoads& t, float* vec, int wave) {
  const uint32_t voff = (uint32_t)fresh_lane_id() * 4;
  const uint32_t soff = (uint32_t)wave * 64 * 4;
  const uint32_t base = lds_addr(vec) + wave * 64 * 4;
  if (g.bias) lds_dma_b32(buffer_rsrc(g.bias + t.n0, TN * 4), voff, soff, base);
  if (g.col_scale) lds_dma_b32(buffer_rsrc(g.col_scale + t.n0, TN * 4), voff, soff, base + 256 * 4);
  if (g.gate) lds_dma_b32(buffer_rsrc(g.gate + t.n0, TN * 4), voff, soff, base + 512 * 4);
  if (g.row_scale) lds_dma_b32(buffer_rsrc(g.row_scale + t.m0, (uint32_t)(t.m_valid * 4)), voff, soff, base + 768 * 4);
}

// Neutral values for the absent epilogue vectors, in both LDS vector buffers: bias -0 (x + -0 == x
// for every x, signed zeros included) and scale 1.
__device__ __forceinline__ void init_vectors(const GemmArgs& g, float (*svec)[kVecFloats], int tid) {
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (!g.bias) svec[b][tid] = -0.0f;
    if (!g.col_scale) svec[b][256 + tid] = 1.0f;
    if (!g.gate) svec[b][512 + tid] = 1.0f;
    if (!g.row_scale) svec[b][768 + tid] = 1.0f;
  }
}

// ------------------------------------------------------------------------------------------------
// Epilogue. The accumulator of tile (i, j) gives lane l token 32 j + (l & 31) of the wave's block and
// features n = 32 i + 8 g + 4 (l >> 5) + q (g, q in 0..3), so the per-element math (scales, bias,
// GELU, bf16 rounding, MX block exponent with one exchange with lane l ^ 32) is lane-local. Stored
// straight from that layout, one store instruction would touch 32 rows; instead each wave stages
// 64 tokens at a time in its own 16 KiB of LDS and stores whole row segments: 16 lanes x 16 bytes
// = one token's 256-byte bf16 segment (8 lanes for the 128-byte e4m3 segment), 8 full cache lines
// per instruction, half as many instructions.
// ------------------------------------------------------------------------------------------------
constexpr int kStageWave = 16384;  // LDS staging bytes per wave

// Buffer resource over `rows` rows of `row_bytes` bytes from p (rows clamped to [0, 64] by the
// caller): the hardware drops stores past the extent and returns zero for loads past it. Offsets stay
// below 64 rows x row_bytes < 2^31 (ldo < 2^22, checked on the host).
// Every input is the same in all lanes (tile, wave and half indices), but the compiler did not prove
// it and wrapped each store through the resource in a loop over distinct resource values
// (readfirstlane, 64-bit compares, exec masking: about a dozen instructions per store); taking the
// address and extent through readfirstlane keeps the resource in scalar registers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* p, int rows, uint32_t row_bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const uint32_t n = __builtin_amdgcn_readfirstlane((uint32_t)rows * row_bytes);
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), (short)0, (int)n,
                                           0x00020000);
}
// 16-byte store through such a resource, non-temporal (cache policy 2): the tile is written once
// and read by the next kernel long after it would have left L2, and streaming it past L2 keeps the
// stores from competing with the operand traffic of the tiles still in their main loops (measured:
// 0.2 ms of 2.7 on the QKV projection).
__device__ __forceinline__ void store_rows_nt16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 d) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{d.x, d.y, d.z, d.w}, r, (int)off, 0, 2);
}

// The gated-residual epilogue's residual rows of one half (64 tokens x the wave's 128 features,
// bf16) into the wave's private 16 KiB residual area by direct-to-LDS loads, so that their latency
// runs under the epilogue's math instead of after it: instruction it lands rows 4 it .. 4 it + 3,
// lane l row 4 it + (l >> 4), 16-byte chunk l & 15, at byte 1024 it + 16 l -- where lane l reads
// it back. Rows past M read zero (the resource ends at row M, as the stores' does).
__device__ __forceinline__ void residual_to_lds(const GemmArgs& g, uint8_t* rarea, int mbase, int nw, int lane) {
  // the tile's row and column pass through an empty asm so that none of this is computed ahead of
  // the k loop and held through it (which spilled registers inside the loop)
  asm volatile("" : "+s"(mbase), "+s"(nw));
  const int rows = max(0, min(64, (int)g.M - mbase));
  const uint32_t rb = (uint32_t)g.ldo * 2;
  // the resource's words through readfirstlane, as in rows_rsrc (the inputs are wave-uniform, which
  // the compiler does not prove, and the load takes the resource in scalar registers)
  const uint64_t base = reinterpret_cast<uint64_t>(g.residual + (size_t)mbase * g.ldo + nw);
  const u32x4 r = {(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)base),
                   (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(base >> 32)) & 0xFFFFu,
                   (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)rows * rb), 0x00020000u};
  const uint32_t voff = (uint32_t)(lane >> 4) * rb + (uint32_t)(lane & 15) * 16;
#pragma unroll
  for (int it = 0; it < 16; ++it) lds_dma_b128(r, voff + (uint32_t)(it * 4) * rb, lds_addr(rarea + it * 1024));
}

// bf16 staging: [64 tokens][256 B], 16-byte chunk index XOR (token & 15) -- the 16 lanes of an LDS
// cycle hit 16 distinct chunks both when writing (16 tokens, one chunk) and reading (one token).
__device__ __forceinline__ int stg16(int tok, int chunk) { return tok * 256 + ((chunk ^ (tok & 15)) << 4); }
// e4m3 staging: [64 tokens][128 B], chunk XOR ((token >> 1) & 7) (two 128-byte rows per bank cycle).
__device__ __forceinline__ int stg8(int tok, int chunk) { return tok * 128 + ((chunk ^ ((tok >> 1) & 7)) << 4); }

// The epilogue vectors of a wave's 128 features in registers: lane (h) needs features
// 32 i + 8 gi + 4 h + q (q = 0..3) of the bias and of the column scales, the same for all 128 tokens,
// so they are read from LDS once per tile instead of once per 16-value block.
template <bool kScaled>
struct EpiVectors {
  float4 bias[4][4];                      // [i][gi]
  float4 cs[kScaled ? 4 : 1][kScaled ? 4 : 1];
};

template <bool kScaled>
__device__ __forceinline__ void load_epi_vectors(const float* vec, int wn, int h, EpiVectors<kScaled>& ev) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int gi = 0; gi < 4; ++gi) {
      const int nl = wn * 128 + i * 32 + gi * 8 + h * 4;
      ev.bias[i][gi] = *reinterpret_cast<const float4*>(vec + nl);
      if constexpr (kScaled) ev.cs[i][gi] = *reinterpret_cast<const float4*>(vec + 256 + nl);
    }
}

// Scaled, biased accumulator values of tile (i, j) for this lane: v = (acc * row_scale) * col_scale
// + bias (absent vectors hold their neutral values, so this is exact without them). Without scale
// vectors (the MX-only projections) x * 1 == x exactly, so the two multiplies are skipped with the
// same result.
template <bool kScaled>
__device__ __forceinline__ void epi_values(const f32x16& a, const EpiVectors<kScaled>& ev, int i, float rsc,
                                           float (&v)[16]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int gi = 0; gi < 4; ++gi) {
    const float4 b = ev.bias[i][gi];
    const float bb[4] = {b.x, b.y, b.z, b.w};
    if constexpr (!kScaled) {
#pragma unroll
      for (int q = 0; q < 4; ++q) v[gi * 4 + q] = a[gi * 4 + q] + bb[q];
    } else {
      const float4 cs = ev.cs[i][gi];
      const float cc[4] = {cs.x, cs.y, cs.z, cs.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) v[gi * 4 + q] = (a[gi * 4 + q] * rsc) * cc[q] + bb[q];
    }
  }
}

// One wave's 128 x 128 block: two halves of 64 tokens (accumulator columns j = 2 hf, 2 hf + 1).
// `stage` is the wave's private LDS staging area; LDS operations of one wave complete in order, so
// the read-back needs no barrier.
// kScaled / kSumsq: row or column scales given / the bf16 epilogue's per-row sums of squares
// requested. They are template parameters so that the epilogue is straight-line code: with runtime
// flags every 16-value block branched, and the LDS reads of its bias and scales were each waited for
// on the spot.
template <int EPI, bool kScaled, bool kSumsq>
__device__ __forceinline__ void epilogue(const GemmArgs& g, const f32x16 (&acc)[4][4], const float* vec, uint8_t* stage,
                                         int m0, int n0, int wm, int wn, uint8_t* rarea = nullptr) {
#pragma clang fp contract(off)
  const int lane = fresh_lane_id();
  const int h = lane >> 5, r32 = lane & 31;
  const int nw = n0 + wn * 128;  // first feature of the wave's block
  // gated residual: `rarea` is 16 KiB of LDS private to the wave that no load targets during the
  // epilogue; the first half's residual rows go there now, the second half's once the first's are read
  if constexpr (EPI == WANMI_EPI_GATED_RESIDUAL) residual_to_lds(g, rarea, m0 + wm * 128, nw, lane);
  EpiVectors<kScaled> ev;
  load_epi_vectors<kScaled>(vec, wn, h, ev);
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    // ---- lane-local math, results into the staging area ----
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * hf + jj;
      const int tok = jj * 32 + r32;  // token within the half
      [[maybe_unused]] uint32_t sbytes = 0;
      // bf16 epilogue with row_sumsq: this lane's part of the token's sum of squares of the rounded
      // outputs over the wave's 128 columns (features 32 i + 8 gi + 4 h + q, in that order)
      [[maybe_unused]] float ss = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v[16];
        epi_values<kScaled>(acc[i][j], ev, i, kScaled ? vec[768 + wm * 128 + j * 32 + r32] : 1.0f, v);
        if constexpr (EPI == WANMI_EPI_GELU_MX) {
          // GELU rounded to bf16 two values per conversion; the block's largest exponent field is
          // that of its largest |y|, taken as the largest (bits & 0x7fff) of the packed bf16 pairs;
          // the codes come from the packed pairs by the scaled conversion
          uint32_t pp[8];
          u16x2 mag = {0, 0};
#pragma unroll
          for (int q = 0; q < 16; q += 2) {
            const uint32_t p = pack_bf16x2(gelu_tanh(v[q]), gelu_tanh(v[q + 1]));
            pp[q / 2] = p;
            mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2, p & 0x7FFF7FFFu));
          }
          int e = (int)(max(mag[0], mag[1]) >> 7);
          e = max_with_lane_xor32(e);  // lanes l and l^32 hold the two halves of the 32-block
          const int sx = max(e - 7, 0);
          const float sc = __uint_as_float((uint32_t)sx << 23);
          sbytes |= (uint32_t)sx << (8 * i);
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            // features 32 i + 8 gi + 4 h .. +3: chunk 2 i + (gi >> 1), byte 8 (gi & 1) + 4 h
            const uint32_t c4 = cvt_e4m3x4_scaled(pp[2 * gi], pp[2 * gi + 1], sc);
            *reinterpret_cast<uint32_t*>(stage + stg8(tok, 2 * i + (gi >> 1)) + 8 * (gi & 1) + 4 * h) = c4;
          }
        } else {
#pragma unroll
          for (int gi = 0; gi < 4; ++gi) {
            float y[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float x = v[gi * 4 + q];
              y[q] = EPI == WANMI_EPI_GELU_BF16 ? gelu_tanh(x) : x;  // gated residual: bf16(v) here
            }
            // features 32 i + 8 gi + 4 h .. +3: chunk 4 i + gi, byte 8 h
            const uint32_t p0 = pack_bf16x2(y[0], y[1]), p1 = pack_bf16x2(y[2], y[3]);
            *reinterpret_cast<uint2*>(stage + stg16(tok, 4 * i + gi) + 8 * h) = make_uint2(p0, p1);
            if constexpr (EPI == WANMI_EPI_BF16) {
              if constexpr (kSumsq) {
                const float b[4] = {bf16_lo(p0), bf16_hi(p0), bf16_lo(p1), bf16_hi(p1)};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                  const float sq = b[q] * b[q];
                  ss = ss + sq;
                }
              }
            }
          }
        }
      }
      if constexpr (EPI == WANMI_EPI_BF16) {
        // the token's sum over the wave's 128 columns: lane h = 0's part, then lane h = 1's
        if (kSumsq && nw < g.sumsq_cols) {
          const float other = __shfl_xor(ss, 32, 64);
          const float tot = h == 0 ? ss + other : other + ss;
          const int m = m0 + wm * 128 + j * 32 + r32;
          if (h == 0 && m < (int)g.M) g.row_sumsq[(uint32_t)m * (uint32_t)g.sumsq_ld + (uint32_t)(nw / 128)] = tot;
        }
      }
      if constexpr (EPI == WANMI_EPI_GELU_MX) {
        const int m = m0 + wm * 128 + j * 32 + r32;
        if (h == 0 && m < (int)g.M)
          __builtin_nontemporal_store(sbytes, reinterpret_cast<uint32_t*>(g.out_scales + (uint32_t)m * (uint32_t)(g.N / 32) +
                                                                         (uint32_t)(nw / 32)));
      }
    }
    // ---- read back whole row segments and store them ----
    // The half's 64 token rows go through a buffer resource whose extent ends at row M: stores to
    // rows past it are dropped and residual loads from them read zero, so there is no per-row branch
    // (with one, the compiler waited for each staging read inside its branch).
    const int mbase = m0 + wm * 128 + hf * 64;
    const int rows = max(0, min(64, (int)g.M - mbase));
    // Loads issued before the epilogue (the next tile's stage 0, when prefetched here) must be
    // complete before the first store: vmcnt counts loads and stores together and stores may finish
    // out of order with loads, so once stores are queued between them and the next tile's stage-1
    // loads, the partial vmcnt wait at the top of the tile would no longer certify stage 0.
    // The gated residual waits here for its half's residual rows too (the second half's were issued
    // before the first half's stores, so only a full wait certifies them).
    if (hf == 0 || EPI == WANMI_EPI_GATED_RESIDUAL) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    if constexpr (EPI == WANMI_EPI_GELU_MX) {
      const uint32_t rb = (uint32_t)g.ldo;  // bytes per output row
      const auto orsrc = rows_rsrc(reinterpret_cast<uint8_t*>(g.out) + (size_t)mbase * rb + nw, rows, rb);
      const int chunk = lane & 7;
      uint4 d[8];
#pragma unroll
      for (int it = 0; it < 8; ++it) d[it] = *reinterpret_cast<const uint4*>(stage + stg8(it * 8 + (lane >> 3), chunk));
#pragma unroll
      for (int it = 0; it < 8; ++it)
        store_rows_nt16(orsrc, (uint32_t)(it * 8 + (lane >> 3)) * rb + (uint32_t)chunk * 16, d[it]);
    } else if constexpr (EPI == WANMI_EPI_GATED_RESIDUAL) {
      // out = bf16(res + bf16(v) * gate), 8 features per lane; the residual rows come from the
      // wave's residual area, where lane l's 16 bytes of row 4 it + (l >> 4) sit at 1024 it + 16 l
      const uint32_t rb = (uint32_t)g.ldo * 2;
      const auto orsrc = rows_rsrc(reinterpret_cast<uint16_t*>(g.out) + (size_t)mbase * g.ldo + nw, rows, rb);
      const int chunk = lane & 15;
      const float4 g0 = *reinterpret_cast<const float4*>(vec + 512 + wn * 128 + chunk * 8);
      const float4 g1 = *reinterpret_cast<const float4*>(vec + 512 + wn * 128 + chunk * 8 + 4);
      const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
      for (int it = 0; it < 16; ++it) {
        const int tok = it * 4 + (lane >> 4);
        const uint4 d = *reinterpret_cast<const uint4*>(stage + stg16(tok, chunk));
        const uint4 rs = *reinterpret_cast<const uint4*>(rarea + it * 1024 + lane * 16);
        const uint32_t dv[4] = {d.x, d.y, d.z, d.w};
        const uint32_t rv[4] = {rs.x, rs.y, rs.z, rs.w};
        uint32_t o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float y0 = bf16_lo(rv[k]) + bf16_lo(dv[k]) * gg[2 * k];
          const float y1 = bf16_hi(rv[k]) + bf16_hi(dv[k]) * gg[2 * k + 1];
          o[k] = pack_bf16x2(y0, y1);
        }
        store_rows_nt16(orsrc, (uint32_t)tok * rb + (uint32_t)chunk * 16, make_uint4(o[0], o[1], o[2], o[3]));
      }
      if (hf == 0) {
        // every read of the area is complete before the second half's rows may land in it
        __builtin_amdgcn_s_waitcnt(waitcnt_lgkm(0));
        residual_to_lds(g, rarea, mbase + 64, nw, lane);
      }
    } else {
      const uint32_t rb = (uint32_t)g.ldo * 2;
      const auto orsrc = rows_rsrc(reinterpret_cast<uint16_t*>(g.out) + (size_t)mbase * g.ldo + nw, rows, rb);
      const int chunk = lane & 15;
#pragma unroll
      for (int b = 0; b < 2; ++b) {  // two batches of 8 reads, then 8 stores
        uint4 d[8];
#pragma unroll
        for (int it = 0; it < 8; ++it)
          d[it] = *reinterpret_cast<const uint4*>(stage + stg16((b * 8 + it) * 4 + (lane >> 4), chunk));
#pragma unroll
        for (int it = 0; it < 8; ++it)
          store_rows_nt16(orsrc, (uint32_t)((b * 8 + it) * 4 + (lane >> 4)) * rb + (uint32_t)chunk * 16, d[it]);
      }
    }
  }
}

// V^T epilogue: the V columns of the fused QKV projection, written in the attention kernel's V^T
// layout. It runs on the transposed accumulator (kSwap: lane l holds feature 32 i + (l & 31) and
// tokens 32 j + 8 g + 4 (l >> 5) + q), so four consecutive tokens of one feature are lane-local. The
// wave's 128 features are one head (the V columns start at a multiple of 256); its tokens become
// columns of the head's 128 rows [d][vt_ld]. Inside each group of 16 the keys are stored in the order
// (0-3, 8-11, 4-7, 12-15) -- the order in which the attention's P registers hand keys to its P V
// MFMA -- so the 4 tokens 8 g + 4 h + q of a lane land in storage slots 4 (2 h + (g & 1)) + q of their
// group: one 8-byte LDS write. Tokens >= M are written as zero. Each half of 64 tokens is staged as
// [128 d][64 slots] bf16 in the wave's LDS area, 16-byte chunks XOR-swizzled by (d >> 1) & 7 so that
// the writes of 32 rows spread over the banks, then stored as whole 128-byte row segments, 8 lanes
// per row; segments at or past vt_ld are dropped.
constexpr int kEpiVt = 100;  // internal epilogue id (wanmi_mxfp8_gemm_qkv only)

__device__ __forceinline__ int vt_chunk(int d, int c16) { return d * 128 + ((c16 ^ ((d >> 1) & 7)) << 4); }

template <bool kScaled>
__device__ __forceinline__ void epilogue_vt(const GemmArgs& g, const f32x16 (&acc)[4][4], const float* vec,
                                            uint8_t* stage, int m0, int n0, int wm, int wn) {
#pragma clang fp contract(off)
  const int lane = fresh_lane_id();
  const int h = lane >> 5, r32 = lane & 31;
  // this lane's feature of each 32-feature fragment: bias and column scale
  float fb[4], fc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    fb[i] = vec[wn * 128 + i * 32 + r32];
    fc[i] = kScaled ? vec[256 + wn * 128 + i * 32 + r32] : 1.0f;
  }
  const int64_t vrow0 = (int64_t)(n0 + wn * 128);  // first V^T row of the wave (head * 128), W rows offset
  const auto vrsrc = rows_rsrc(g.vt + vrow0 * g.vt_ld, 128, (uint32_t)g.vt_ld * 2);
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * hf + jj;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int tok0 = wm * 128 + j * 32 + 8 * gq + 4 * h;  // first of the 4 tokens, within the tile
        float rs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (kScaled) {
          const float4 r4 = *reinterpret_cast<const float4*>(vec + 768 + tok0);
          rs[0] = r4.x, rs[1] = r4.y, rs[2] = r4.z, rs[3] = r4.w;
        }
        const int live = (int)g.M - (m0 + tok0);  // tokens q < live are inside M
        const int c16 = 2 * (2 * jj + (gq >> 1)) + h;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float y[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float a = acc[i][j][gq * 4 + q];
            const float v = kScaled ? (a * rs[q]) * fc[i] + fb[i] : a + fb[i];
            y[q] = q < live ? v : 0.0f;
          }
          const int d = i * 32 + r32;
          *reinterpret_cast<uint2*>(stage + vt_chunk(d, c16) + (gq & 1) * 8) =
              make_uint2(pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3]));
        }
      }
    }
    const int mbase = m0 + wm * 128 + hf * 64;
    if (hf == 0) __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // loads before stores, as in epilogue()
    const int chunk = lane & 7;
    const uint32_t col_bytes = (uint32_t)(mbase + chunk * 8) * 2;
    const bool in_row = mbase + chunk * 8 < (int)g.vt_ld;
#pragma unroll
    for (int b = 0; b < 2; ++b) {  // two batches of 8 reads, then 8 stores
      uint4 dv[8];
#pragma unroll
      for (int it = 0; it < 8; ++it)
        dv[it] = *reinterpret_cast<const uint4*>(stage + vt_chunk((b * 8 + it) * 8 + (lane >> 3), chunk));
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const uint32_t d = (uint32_t)((b * 8 + it) * 8 + (lane >> 3));
        // an offset past the resource's extent drops the store (segments at or past vt_ld);
        // non-temporal, as the other epilogues' outputs (through L2 the QKV pair ran 0.5% slower)
        const uint32_t off = in_row ? d * (uint32_t)g.vt_ld * 2 + col_bytes : 0xFFFFFFF0u;
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{dv[it].x, dv[it].y, dv[it].z, dv[it].w}, vrsrc, (int)off, 0, 2);
      }
    }
  }
}

// K not a multiple of 512: a simple double-buffered loop that issues the next stage's loads after all
// reads of the current one (the pipelined loop, mxfp8_gemm_ring_kernel below, needs whole scale
// groups).
template <int EPI>
__global__ __launch_bounds__(256, 1) void mxfp8_gemm_kernel(GemmArgs g) {
#pragma clang fp contract(off)
  constexpr bool kSwap = EPI == kEpiVt;  // the V^T epilogue wants the transposed accumulator
  __shared__ __attribute__((aligned(16))) uint8_t smem0[kStageBytes];
  __shared__ __attribute__((aligned(16))) uint8_t smem1[kStageBytes];
  __shared__ __attribute__((aligned(16))) uint32_t ssc[2][2 * 256 * 4];  // scale groups, double-buffered
  __shared__ __attribute__((aligned(16))) float svec[2][kVecFloats];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave >> 1, wm = wave & 1;
  const int h = lane >> 5;
  const int r32 = lane & 31;
  const int KT = (int)(g.K / BK);
  const int total = g.tiles_m * g.tiles_n;
  // Prefetching the next tile before the epilogue would make the gated-residual epilogue's own
  // residual loads wait behind those loads (the wait counter is in order), so that epilogue
  // prefetches after.
  constexpr bool kPrefetchBeforeEpilogue = EPI != WANMI_EPI_GATED_RESIDUAL;
  // The epilogue stages its output in smem1, so only stage 0 of the next tile (smem0, with the
  // first scale group and the epilogue vectors) may be loaded before or during it.
  auto prefetch0 = [&](const TileLoads& tl, float* vec) {
    issue_vectors(g, tl, vec, wave);
    issue_scales(g, tl, 0, ssc[0], wave);
    issue_codes(g, tl, 0, smem0, wave);
  };

  int v = blockIdx.x;
  init_vectors(g, svec, tid);  // published by the barrier at the top of the tile loop
  prefetch0(tile_loads(g, v), svec[0]);
  int vb = 0;

  f32x16 acc[4][4];
  for (;;) {
    // tile state is recomputed per tile (cheap scalar work) rather than carried across the epilogue
    const TileLoads t = tile_loads(g, v);
    // this tile's stage 0, scales and vectors have landed
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int kt = 0; kt < KT; ++kt) {
      uint8_t* cur = (kt & 1) ? smem1 : smem0;
      uint8_t* nxt = (kt & 1) ? smem0 : smem1;
      const uint32_t* sc = ssc[(kt / kScaleGroup) & 1];
      // nobody reads nxt, nor the other scale buffer, since the last barrier
      if (kt + 1 < KT) {
        if ((kt + 1) % kScaleGroup == 0) issue_scales(g, t, (kt + 1) / kScaleGroup, ssc[((kt + 1) / kScaleGroup) & 1], wave);
        issue_codes(g, t, kt + 1, nxt, wave);
      }
      SliceOperands op;
      const uint32_t sl = scale_lane_offset();
      read_slice(cur, sc, kt % kScaleGroup, 0, op, wn, wm, h, r32, sl);
      mfma_rows<0, 4, kSwap>(op, acc);
      read_slice(cur, sc, kt % kScaleGroup, 1, op, wn, wm, h, r32, sl);
      mfma_rows<0, 4, kSwap>(op, acc);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }

    // Every wave is past its last LDS operand read of this tile once all have passed a barrier, and
    // the zero-fill loads past the end of K (which target the stage buffers) are complete after
    // vmcnt(0); then smem0 may take the next tile's stage 0 and smem1 serves as staging.
    const int m0 = (int)t.m0, n0 = (int)t.n0;
    const int vn = v + (int)gridDim.x;
    const bool has_next = vn < total;
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    if (kPrefetchBeforeEpilogue && has_next) prefetch0(tile_loads(g, vn), svec[vb ^ 1]);
    {
      uint8_t* stage = smem1 + wave * kStageWave;
      // the gated residual's rows: smem0, which that epilogue's tile only prefetches into after it
      uint8_t* rarea = smem0 + wave * kStageWave;
      const bool scaled = g.row_scale || g.col_scale;
      if constexpr (EPI == kEpiVt) {
        if (scaled) epilogue_vt<true>(g, acc, svec[vb], stage, m0, n0, wm, wn);
        else epilogue_vt<false>(g, acc, svec[vb], stage, m0, n0, wm, wn);
      } else if constexpr (EPI == WANMI_EPI_BF16) {
        if (g.row_sumsq) {
          if (scaled) epilogue<EPI, true, true>(g, acc, svec[vb], stage, m0, n0, wm, wn);
          else epilogue<EPI, false, true>(g, acc, svec[vb], stage, m0, n0, wm, wn);
        } else {
          if (scaled) epilogue<EPI, true, false>(g, acc, svec[vb], stage, m0, n0, wm, wn);
          else epilogue<EPI, false, false>(g, acc, svec[vb], stage, m0, n0, wm, wn);
        }
      } else {
        if (scaled) epilogue<EPI, true, false>(g, acc, svec[vb], stage, m0, n0, wm, wn, rarea);
        else epilogue<EPI, false, false>(g, acc, svec[vb], stage, m0, n0, wm, wn, rarea);
      }
    }
    if (!has_next) break;
    __syncthreads();  // every wave is done with its staging area in smem1
    if (!kPrefetchBeforeEpilogue) prefetch0(tile_loads(g, vn), svec[vb ^ 1]);
    v = vn;
    vb ^= 1;
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load may still target LDS when the workgroup retires
}

// ------------------------------------------------------------------------------------------------
// The pipelined k loop (K a multiple of 512), with its loads split over both phases of a stage.
// A stage is two phases of 16 MFMAs, each split into four fragment rows (4 MFMAs each) with the LDS
// reads of one fragment row of the next slice issued before them (phase A: MFMAs on slice 0, reads
// of slice 1; phase B: MFMAs on slice 1, reads of slice 0 of the next stage), and the stage's loads
// two stages ahead spread one at a time between the MFMAs; the scheduling barriers keep the compiler
// from regrouping them (it otherwise moves MFMAs across the stage's barrier and clusters the reads).
// All 16 of a stage's loads in phase B (the two-buffer form) asked for 64 B/clk per CU during that
// phase, above what direct-to-LDS streaming sustains, and stretched it.
// LDS: the weight codes of a stage in two 16 KiB halves (rows 0-127, 128-255) on a ring of five half
// slots, the activation codes in two 32 KiB slots, the scale groups as before; 160 KiB. Half k = 2 S + h of stage S sits in half slot
// k % 5, so the slot of stage S+2's first half (k = 2S+4) held stage S-1's second half, free since
// the barrier of stage S-1: those 4 loads per wave go out in phase A of stage S, and stage S+2's
// second half (the slot of stage S's first half) and its activations (stage S's activation slot),
// 12 loads per wave, in phase B after the barrier. A wave's MFMA weight rows are one half (wn), so
// its reads address one half slot. The epilogue vectors have no buffer of their own: at the tile's
// last scale-group load (stage KT-2, for the group past its end) the scale loads are masked off and
// wave w fetches vector w (bias, column scale, gate, row scale; 1 KiB each) into the scale buffer
// that group would have used; the next tile's scale groups start in the other one.
// ------------------------------------------------------------------------------------------------
constexpr int kHalfBytes = 128 * BK;  // 16 KiB: 128 weight rows of one stage
constexpr int kActBytes = TM * BK;    // 32 KiB: 256 token rows of one stage
// Neutral epilogue vectors, loaded in place of an absent one: bias -0, scales and gate 1.
#define WANMI_R8(x) x, x, x, x, x, x, x, x
#define WANMI_R64(x) WANMI_R8(x), WANMI_R8(x), WANMI_R8(x), WANMI_R8(x), WANMI_R8(x), WANMI_R8(x), WANMI_R8(x), WANMI_R8(x)
__device__ const float kNeutralNegZero[256] = {WANMI_R64(-0.0f), WANMI_R64(-0.0f), WANMI_R64(-0.0f), WANMI_R64(-0.0f)};
__device__ const float kNeutralOne[256] = {WANMI_R64(1.0f), WANMI_R64(1.0f), WANMI_R64(1.0f), WANMI_R64(1.0f)};
#undef WANMI_R64
#undef WANMI_R8

// Descriptor of wave w's epilogue vector for tile t (extent: the row scale stops at row M).
__device__ __forceinline__ u32x4 vector_rsrc(const GemmArgs& g, const TileLoads& t, int wave) {
  const float* p = wave == 0 ? (g.bias ? g.bias + t.n0 : kNeutralNegZero)
                 : wave == 1 ? (g.col_scale ? g.col_scale + t.n0 : kNeutralOne)
                 : wave == 2 ? (g.gate ? g.gate + t.n0 : kNeutralOne)
                             : (g.row_scale ? g.row_scale + t.m0 : kNeutralOne);
  const uint32_t bytes = (wave == 3 && g.row_scale) ? (uint32_t)(t.m_valid * 4) : 1024u;
  return buffer_rsrc(p, bytes);
}

// A direct-to-LDS load under an all-or-nothing lane mask (exec set and restored inside the block),
// so that a load is switched on or off without a branch. Five wait states as lds_dma_b128.
__device__ __forceinline__ void lds_dma_b128_masked(u32x4 rsrc, uint32_t voff, uint32_t lds, bool on) {
  uint64_t saved;
  const uint32_t m = __builtin_amdgcn_readfirstlane(on ? ~0u : 0u);  // exec_lo and exec_hi alike
  asm volatile("s_mov_b64 %0, exec\n\ts_mov_b32 exec_lo, %3\n\ts_mov_b32 exec_hi, %3\n\ts_nop 4\n\t"
               "buffer_load_dwordx4 %1, %2, 0 offen lds\n\ts_mov_b64 exec, %0"
               : "=&s"(saved)
               : "v"(voff), "s"(rsrc), "s"(m), "{m0}"(lds)
               : "memory");
}

// After the barrier of stage S = 4G + 2: the scales of group G + 1 (2 loads per wave) if the tile
// has that group, else the tile's epilogue vectors (1 load per wave: vector w) into the buffer that
// group would have used. Both are issued, one of them masked off.
__device__ __forceinline__ void issue_scales_or_vectors(const GemmArgs& g, const TileLoads& t, int grp, uint32_t* sc,
                                                        int wave, bool more) {
  const uint32_t KB = (uint32_t)(g.K / 32);
  const uint32_t lane = (uint32_t)fresh_lane_id();
  const uint32_t v = (uint32_t)(wave * 64 + lane) * KB + (uint32_t)grp * 16;
  const uint32_t ls = lds_addr(sc) + wave * 64 * 16;
  lds_dma_b128_masked(t.ws, v, ls, more);
  lds_dma_b128_masked(t.as, v, ls + TN * 16, more);
  lds_dma_b128_masked(vector_rsrc(g, t, wave), lane * 16, lds_addr(sc) + wave * 1024, !more);
}

// One direct-to-LDS load of weight half hh, row group p (rows 128 hh + 8 p .. + 7) of stage kt into
// the half slot at `dst`; of activation row group p (rows 8 p .. + 7) into the slot at `dst`.
template <bool kHot>
__device__ __forceinline__ void w_half_dma(const GemmArgs& g, const TileLoads& t, const DmaLanes& dl, int kt, int hh,
                                           int p, uint32_t dst, bool valid) {
  const uint32_t off = ((p & 1) ? dl.wo : dl.we) + (uint32_t)(128 * hh + 8 * p) * (uint32_t)g.K + (uint32_t)kt * BK;
  if constexpr (kHot)
    lds_dma_b128_hot(maybe_empty(t.w, valid), off, dst + (uint32_t)(8 * p * BK));
  else
    lds_dma_b128(maybe_empty(t.w, valid), off, dst + (uint32_t)(8 * p * BK));
}
template <bool kHot>
__device__ __forceinline__ void act_dma(const GemmArgs& g, const TileLoads& t, const DmaLanes& dl, int kt, int p,
                                        uint32_t dst, bool valid) {
  const uint32_t off = ((p & 1) ? dl.ao : dl.ae) + (uint32_t)(8 * p) * (uint32_t)g.lda + (uint32_t)kt * BK;
  if constexpr (kHot)
    lds_dma_b128_hot(maybe_empty(t.a, valid), off, dst + (uint32_t)(8 * p * BK));
  else
    lds_dma_b128(maybe_empty(t.a, valid), off, dst + (uint32_t)(8 * p * BK));
}

// All 16 loads of stage kt outside the k loop: wave w takes weight row groups 4w .. 4w+3 of both
// halves and activation row groups 8w .. 8w+7.
__device__ __forceinline__ void issue_stage_r(const GemmArgs& g, const TileLoads& t, int kt, uint32_t h0, uint32_t h1,
                                              uint32_t act, int wave) {
  const DmaLanes dl = dma_lanes(g);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    w_half_dma<false>(g, t, dl, kt, 0, 4 * wave + i, h0, true);
    w_half_dma<false>(g, t, dl, kt, 1, 4 * wave + i, h1, true);
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) act_dma<false>(g, t, dl, kt, 8 * wave + i, act, true);
}

// Phase A row I: reads of slice 1 of the stage, 4 MFMAs, and weight row group 4w + I of half 0 of
// stage kt (two stages ahead) after the first MFMA.
template <int I, bool kSwap>
__device__ __forceinline__ void phase_a_row_r(const uint8_t* wb, const uint8_t* ab, const uint32_t* sc, int q,
                                              SliceOperands& nxt, const SliceOperands& cur, f32x16 (&acc)[4][4], int wn,
                                              int wm, int h, int r32, uint32_t sl, const GemmArgs& g,
                                              const TileLoads& t, const DmaLanes& dl, int kt, uint32_t h0, int wave,
                                              bool valid) {
  read_slice_r<I, I + 1>(wb, ab, sc, q, 1, nxt, wn, wm, h, r32, sl);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[I][j] = mfma_tile<kSwap>(cur.w[I], cur.a[j], acc[I][j], cur.ws[I], cur.as[j]);
    if (j == 0) w_half_dma<true>(g, t, dl, kt, 0, 4 * wave + I, h0, valid);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Phase B row I: reads of slice 0 of the next stage, 4 MFMAs, and three loads of stage kt: weight
// row group 4w + I of half 1 and activation row groups 8w + 2I, 8w + 2I + 1.
template <int I, bool kSwap>
__device__ __forceinline__ void phase_b_row_r(const uint8_t* wb, const uint8_t* ab, const uint32_t* sc, int q,
                                              SliceOperands& nxt, const SliceOperands& cur, f32x16 (&acc)[4][4], int wn,
                                              int wm, int h, int r32, uint32_t sl, const GemmArgs& g,
                                              const TileLoads& t, const DmaLanes& dl, int kt, uint32_t h1,
                                              uint32_t act, int wave, bool valid) {
  read_slice_r<I, I + 1>(wb, ab, sc, q, 0, nxt, wn, wm, h, r32, sl);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    acc[I][j] = mfma_tile<kSwap>(cur.w[I], cur.a[j], acc[I][j], cur.ws[I], cur.as[j]);
    if (j == 0) w_half_dma<true>(g, t, dl, kt, 1, 4 * wave + I, h1, valid);
    if (j == 1) act_dma<true>(g, t, dl, kt, 8 * wave + 2 * I, act, valid);
    if (j == 2) act_dma<true>(g, t, dl, kt, 8 * wave + 2 * I + 1, act, valid);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int EPI>
__global__ __launch_bounds__(256, 1) void mxfp8_gemm_ring_kernel(GemmArgs g) {
#pragma clang fp contract(off)
  constexpr bool kSwap = EPI == kEpiVt;
  __shared__ __attribute__((aligned(16))) uint8_t sWh[5][kHalfBytes];
  __shared__ __attribute__((aligned(16))) uint8_t sAct[2][kActBytes];
  __shared__ __attribute__((aligned(16))) uint32_t ssc[2][2 * 256 * 4];  // scale groups; the tile's vectors at its end

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave >> 1, wm = wave & 1;
  const int h = lane >> 5;
  const int r32 = lane & 31;
  const int KT = (int)(g.K / BK);  // a multiple of 4
  const int total = g.tiles_m * g.tiles_n;
  constexpr bool kPrefetchBeforeEpilogue = EPI != WANMI_EPI_GATED_RESIDUAL;
  auto hs = [&](int k) { return lds_addr(sWh[k % 5]); };
  // Each tile starts with stage 0's halves in slots 0, 1 and stage 1's in 2, 3; activations of
  // stage S in slot S % 2. Scale group G of a tile uses buffer (G + par) & 1.
  auto prefetch0 = [&](const TileLoads& tl, int par) {
    issue_scales(g, tl, 0, ssc[par & 1], wave);
    issue_stage_r(g, tl, 0, hs(0), hs(1), lds_addr(sAct[0]), wave);
  };
  auto prefetch1 = [&](const TileLoads& tl) { issue_stage_r(g, tl, 1, hs(2), hs(3), lds_addr(sAct[1]), wave); };

  int v = blockIdx.x;
  int par = 0;
  prefetch0(tile_loads(g, v), par);
  prefetch1(tile_loads(g, v));

  f32x16 acc[4][4];
  for (;;) {
    const TileLoads t = tile_loads(g, v);
    const int vpar = ((KT >> 2) + par) & 1;  // scale buffer that takes this tile's epilogue vectors
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kCodeLoads));
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    // Entering stage S, opA holds slice 0 of S. Phase A: slice-0 MFMAs, slice-1 reads of S, stage
    // S+2's first weight half loaded. Barrier after this wave's reads of S and its loads of S+1 are
    // complete (outstanding: the 4 loads just issued). Phase B: slice-1 MFMAs, slice-0 reads of S+1,
    // stage S+2's second weight half and activations loaded. After the barrier of stage 4G+2 the
    // scales of group G+1, or at the tile's last group its epilogue vectors.
#define WANMI_GEMM_RSTAGE(S, ACT_CUR, ACT_OTH, SC_CUR, Q_CUR, SC_NXT, Q_NXT, WITH_SCALES)                      \
  do {                                                                                                  \
    const int k0_ = 2 * (S);                                                                            \
    const bool more_ = (S) + 2 < KT;                                                                    \
    const int ktn_ = more_ ? (S) + 2 : 0;                                                               \
    const uint8_t* wcur_ = sWh[(k0_ + wn) % 5];                                                         \
    const uint8_t* wnxt_ = sWh[(k0_ + 2 + wn) % 5];                                                     \
    const uint32_t h0_ = hs(k0_ + 4), h1_ = hs(k0_ + 5);                                                \
    phase_a_row_r<0, kSwap>(wcur_, ACT_CUR, SC_CUR, Q_CUR, opB, opA, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h0_, wave, more_); \
    phase_a_row_r<1, kSwap>(wcur_, ACT_CUR, SC_CUR, Q_CUR, opB, opA, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h0_, wave, more_); \
    phase_a_row_r<2, kSwap>(wcur_, ACT_CUR, SC_CUR, Q_CUR, opB, opA, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h0_, wave, more_); \
    phase_a_row_r<3, kSwap>(wcur_, ACT_CUR, SC_CUR, Q_CUR, opB, opA, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h0_, wave, more_); \
    __builtin_amdgcn_s_waitcnt(waitcnt_lgkm(0));                                                        \
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(4));                                                          \
    __syncthreads();                                                                                    \
    if (WITH_SCALES)                                                                                    \
      issue_scales_or_vectors(g, t, ((S) + 2) / kScaleGroup, ssc[((((S) + 2) / kScaleGroup) + par) & 1], wave, more_); \
    phase_b_row_r<0, kSwap>(wnxt_, ACT_OTH, SC_NXT, Q_NXT, opA, opB, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h1_, lds_addr(ACT_CUR), wave, more_); \
    phase_b_row_r<1, kSwap>(wnxt_, ACT_OTH, SC_NXT, Q_NXT, opA, opB, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h1_, lds_addr(ACT_CUR), wave, more_); \
    phase_b_row_r<2, kSwap>(wnxt_, ACT_OTH, SC_NXT, Q_NXT, opA, opB, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h1_, lds_addr(ACT_CUR), wave, more_); \
    phase_b_row_r<3, kSwap>(wnxt_, ACT_OTH, SC_NXT, Q_NXT, opA, opB, acc, wn, wm, h, r32, sl, g, t, dl, ktn_, h1_, lds_addr(ACT_CUR), wave, more_); \
  } while (0)

    {
      const DmaLanes dl = dma_lanes(g);
      const uint32_t sl = scale_lane_offset();
      SliceOperands opA, opB;
      read_slice_r(sWh[wn], sAct[0], ssc[par & 1], 0, 0, opA, wn, wm, h, r32, sl);
      for (int kt = 0; kt < KT; kt += 4) {
        const int sg = ((kt / kScaleGroup) + par) & 1;
        WANMI_GEMM_RSTAGE(kt, sAct[0], sAct[1], ssc[sg], 0, ssc[sg], 1, false);
        WANMI_GEMM_RSTAGE(kt + 1, sAct[1], sAct[0], ssc[sg], 1, ssc[sg], 2, false);
        WANMI_GEMM_RSTAGE(kt + 2, sAct[0], sAct[1], ssc[sg], 2, ssc[sg], 3, true);
        WANMI_GEMM_RSTAGE(kt + 3, sAct[1], sAct[0], ssc[sg], 3, ssc[sg ^ 1], 0, false);
      }
    }
#undef WANMI_GEMM_RSTAGE

    // Every wave is past its last LDS read of the tile after a barrier, and the loads past the end
    // of K and the vectors are complete after vmcnt(0). The next tile's stage 0 then goes to half
    // slots 0-1 and activation slot 0, its first scale group to the buffer the vectors are not in;
    // the epilogue stages waves 0-1 in activation slot 1 and waves 2-3 in half slots 2-3, where the
    // next tile's stage 1 is loaded after it.
    const float* vec = reinterpret_cast<const float*>(ssc[vpar]);
    const int m0 = (int)t.m0, n0 = (int)t.n0;
    const int vn = v + (int)gridDim.x;
    const bool has_next = vn < total;
    const int par_n = vpar ^ 1;
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    __syncthreads();
    if (kPrefetchBeforeEpilogue && has_next) prefetch0(tile_loads(g, vn), par_n);
    {
      uint8_t* stage = wave < 2 ? sAct[1] + wave * kStageWave : sWh[wave];
      // the gated residual's rows: activation slot 0 and half slots 0-1, which that epilogue's tile
      // only prefetches into after it
      uint8_t* rarea = wave < 2 ? sAct[0] + wave * kStageWave : sWh[wave - 2];
      const bool scaled = g.row_scale || g.col_scale;
      if constexpr (EPI == kEpiVt) {
        if (scaled) epilogue_vt<true>(g, acc, vec, stage, m0, n0, wm, wn);
        else epilogue_vt<false>(g, acc, vec, stage, m0, n0, wm, wn);
      } else if constexpr (EPI == WANMI_EPI_BF16) {
        if (g.row_sumsq) {
          if (scaled) epilogue<EPI, true, true>(g, acc, vec, stage, m0, n0, wm, wn);
          else epilogue<EPI, false, true>(g, acc, vec, stage, m0, n0, wm, wn);
        } else {
          if (scaled) epilogue<EPI, true, false>(g, acc, vec, stage, m0, n0, wm, wn);
          else epilogue<EPI, false, false>(g, acc, vec, stage, m0, n0, wm, wn);
        }
      } else {
        if (scaled) epilogue<EPI, true, false>(g, acc, vec, stage, m0, n0, wm, wn, rarea);
        else epilogue<EPI, false, false>(g, acc, vec, stage, m0, n0, wm, wn, rarea);
      }
    }
    if (!has_next) break;
    __syncthreads();  // every wave is done with its staging area and the vectors
    if (!kPrefetchBeforeEpilogue) prefetch0(tile_loads(g, vn), par_n);
    prefetch1(tile_loads(g, vn));
    v = vn;
    par = par_n;
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load may still target LDS when the workgroup retires
}

// kPipelined (K a multiple of 512): the pipelined ring kernel; otherwise the simple loop.
template <bool kPipelined>
static void launch_gemm(int epilogue, dim3 grid, hipStream_t stream, const GemmArgs& g) {
  if constexpr (kPipelined) {
    switch (epilogue) {
      case WANMI_EPI_BF16: hipLaunchKernelGGL((mxfp8_gemm_ring_kernel<WANMI_EPI_BF16>), grid, dim3(256), 0, stream, g); break;
      case WANMI_EPI_GELU_MX: hipLaunchKernelGGL((mxfp8_gemm_ring_kernel<WANMI_EPI_GELU_MX>), grid, dim3(256), 0, stream, g); break;
      case WANMI_EPI_GELU_BF16: hipLaunchKernelGGL((mxfp8_gemm_ring_kernel<WANMI_EPI_GELU_BF16>), grid, dim3(256), 0, stream, g); break;
      case kEpiVt: hipLaunchKernelGGL((mxfp8_gemm_ring_kernel<kEpiVt>), grid, dim3(256), 0, stream, g); break;
      default: hipLaunchKernelGGL((mxfp8_gemm_ring_kernel<WANMI_EPI_GATED_RESIDUAL>), grid, dim3(256), 0, stream, g); break;
    }
  } else {
    switch (epilogue) {
      case WANMI_EPI_BF16: hipLaunchKernelGGL((mxfp8_gemm_kernel<WANMI_EPI_BF16>), grid, dim3(256), 0, stream, g); break;
      case WANMI_EPI_GELU_MX: hipLaunchKernelGGL((mxfp8_gemm_kernel<WANMI_EPI_GELU_MX>), grid, dim3(256), 0, stream, g); break;
      case WANMI_EPI_GELU_BF16: hipLaunchKernelGGL((mxfp8_gemm_kernel<WANMI_EPI_GELU_BF16>), grid, dim3(256), 0, stream, g); break;
      case kEpiVt: hipLaunchKernelGGL((mxfp8_gemm_kernel<kEpiVt>), grid, dim3(256), 0, stream, g); break;
      default: hipLaunchKernelGGL((mxfp8_gemm_kernel<WANMI_EPI_GATED_RESIDUAL>), grid, dim3(256), 0, stream, g); break;
    }
  }
}

}  // namespace wanmi

namespace wanmi {
static int gemm_impl(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes, const uint8_t* w_scales,
                     const float* row_scale, const float* col_scale, const float* bias, int64_t M, int64_t N,
                     int64_t K, int64_t lda, int epilogue, void* out, int64_t ldo, uint8_t* out_scales,
                     const void* residual, const float* gate, float* row_sumsq, int64_t sumsq_cols, int64_t sumsq_ld,
                     void* vt, int64_t vt_ld, void* stream) {
  WANMI_REQUIRE(M >= 0 && N > 0 && K > 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm: bad sizes M=%lld N=%lld K=%lld",
                (long long)M, (long long)N, (long long)K);
  WANMI_REQUIRE(N % TN == 0, WANMI_ERR_UNSUPPORTED, "wanmi_mxfp8_gemm: N=%lld must be a multiple of %d",
                (long long)N, TN);
  WANMI_REQUIRE(K % BK == 0, WANMI_ERR_UNSUPPORTED, "wanmi_mxfp8_gemm: K=%lld must be a multiple of %d",
                (long long)K, BK);
  WANMI_REQUIRE((epilogue >= WANMI_EPI_BF16 && epilogue <= WANMI_EPI_GATED_RESIDUAL) || epilogue == kEpiVt,
                WANMI_ERR_ARG, "wanmi_mxfp8_gemm: unknown epilogue %d", epilogue);
  WANMI_REQUIRE(lda >= K && lda % 16 == 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm: lda=%lld must be >= K and a multiple of 16",
                (long long)lda);
  const bool to_vt = epilogue == kEpiVt;
  WANMI_REQUIRE(to_vt || (ldo >= N && ldo % 16 == 0), WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: ldo=%lld must be >= N and a multiple of 16", (long long)ldo);
  if (M == 0) return WANMI_OK;
  WANMI_REQUIRE(a_codes && a_scales && w_codes && w_scales && (to_vt ? vt != nullptr : out != nullptr), WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: null operand");
  WANMI_REQUIRE(epilogue != WANMI_EPI_GELU_MX || out_scales, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: GELU_MX epilogue needs out_scales");
  WANMI_REQUIRE(epilogue != WANMI_EPI_GATED_RESIDUAL || (residual && gate), WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: gated-residual epilogue needs residual and gate");
  WANMI_REQUIRE(((uintptr_t)a_codes % 16) == 0 && ((uintptr_t)w_codes % 16) == 0 &&
                    ((uintptr_t)a_scales % 4) == 0 && ((uintptr_t)w_scales % 4) == 0 &&
                    ((uintptr_t)out % 16) == 0 && (!out_scales || ((uintptr_t)out_scales % 4) == 0) &&
                    (!bias || ((uintptr_t)bias % 16) == 0) &&
                    (!col_scale || ((uintptr_t)col_scale % 16) == 0) &&
                    (!gate || ((uintptr_t)gate % 16) == 0) && (!residual || ((uintptr_t)residual % 16) == 0) &&
                    ((uintptr_t)vt % 16) == 0,
                WANMI_ERR_ARG, "wanmi_mxfp8_gemm: misaligned operand");
  const int64_t tiles = (N / TN) * ((M + TM - 1) / TM);
  WANMI_REQUIRE(tiles < (1LL << 31), WANMI_ERR_ARG, "wanmi_mxfp8_gemm: problem too large");
  WANMI_REQUIRE(to_vt || (M * ldo < (1LL << 32) && M < (1LL << 31)), WANMI_ERR_UNSUPPORTED,
                "wanmi_mxfp8_gemm: M=%lld x ldo=%lld output elements exceed 32-bit offsets", (long long)M, (long long)ldo);
  WANMI_REQUIRE(!to_vt || (vt_ld >= M && vt_ld % 64 == 0 && 128 * vt_ld * 2 < (1LL << 31)), WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: vt_ld=%lld must be >= M, a multiple of 64 and below 2^23", (long long)vt_ld);
  // per-tile buffer offsets are 32-bit; this also keeps K and lda below 2^23 for the 24-bit
  // multiplies of the load offsets
  WANMI_REQUIRE(TN * K < (1LL << 31) && TM * lda < (1LL << 31), WANMI_ERR_UNSUPPORTED,
                "wanmi_mxfp8_gemm: K=%lld / lda=%lld too large", (long long)K, (long long)lda);
  // the epilogue's store resources span 64 output rows with 32-bit offsets
  WANMI_REQUIRE(to_vt || ldo < (1LL << 22), WANMI_ERR_UNSUPPORTED, "wanmi_mxfp8_gemm: ldo=%lld too large", (long long)ldo);

  GemmArgs g;
  g.a = a_codes;
  g.a_scales = a_scales;
  g.w = w_codes;
  g.w_scales = w_scales;
  g.row_scale = row_scale;
  g.col_scale = col_scale;
  g.bias = bias;
  g.residual = static_cast<const uint16_t*>(residual);
  g.gate = epilogue == WANMI_EPI_GATED_RESIDUAL ? gate : nullptr;
  g.out = out;
  g.out_scales = out_scales;
  g.row_sumsq = row_sumsq;
  g.sumsq_cols = row_sumsq ? sumsq_cols : 0;
  g.sumsq_ld = sumsq_ld;
  g.vt = static_cast<uint16_t*>(vt);
  g.vt_ld = vt_ld;
  g.M = M;
  g.N = N;
  g.K = K;
  g.lda = lda;
  g.ldo = ldo;
  g.tiles_m = (int)((M + TM - 1) / TM);
  g.tiles_n = (int)(N / TN);
  // persistent: one workgroup per CU (the LDS footprint allows no second one)
  const int cus = device_cu_count();
  WANMI_REQUIRE(cus > 0, WANMI_ERR_HIP, "wanmi_mxfp8_gemm: cannot query the device's compute units");
  const dim3 grid((unsigned)std::min<int64_t>(tiles, cus));
  if ((K / BK) % 4 == 0)
    launch_gemm<true>(epilogue, grid, (hipStream_t)stream, g);
  else
    launch_gemm<false>(epilogue, grid, (hipStream_t)stream, g);
  return check_launch("wanmi_mxfp8_gemm");
}
}  // namespace wanmi

extern "C" int wanmi_mxfp8_gemm(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                                const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                                const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda,
                                int epilogue, void* out, int64_t ldo, uint8_t* out_scales,
                                const void* residual, const float* gate, void* stream) {
  wanmi::clear_error();
  WANMI_REQUIRE(epilogue >= WANMI_EPI_BF16 && epilogue <= WANMI_EPI_GATED_RESIDUAL, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm: unknown epilogue %d", epilogue);
  return wanmi::gemm_impl(a_codes, a_scales, w_codes, w_scales, row_scale, col_scale, bias, M, N, K, lda, epilogue,
                          out, ldo, out_scales, residual, gate, nullptr, 0, 0, nullptr, 0, stream);
}

extern "C" int wanmi_mxfp8_gemm_rowsumsq(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                                         const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                                         const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda, void* out,
                                         int64_t ldo, float* row_sumsq, int64_t sumsq_cols, void* stream) {
  using namespace wanmi;
  clear_error();
  // no rows: nothing is written, and an empty row_sumsq may have no storage
  WANMI_REQUIRE(M == 0 || (row_sumsq && ((uintptr_t)row_sumsq % 4) == 0), WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm_rowsumsq: row_sumsq must be a 4-byte aligned pointer");
  WANMI_REQUIRE(sumsq_cols >= 0 && sumsq_cols <= N && sumsq_cols % 128 == 0, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm_rowsumsq: sumsq_cols=%lld must be a multiple of 128 in [0, N]", (long long)sumsq_cols);
  return gemm_impl(a_codes, a_scales, w_codes, w_scales, row_scale, col_scale, bias, M, N, K, lda, WANMI_EPI_BF16, out,
                   ldo, nullptr, nullptr, nullptr, row_sumsq, sumsq_cols, N / 128, nullptr, 0, stream);
}

extern "C" int wanmi_mxfp8_gemm_qkv(const uint8_t* a_codes, const uint8_t* a_scales, const uint8_t* w_codes,
                                    const uint8_t* w_scales, const float* row_scale, const float* col_scale,
                                    const float* bias, int64_t M, int64_t N, int64_t K, int64_t lda, void* out,
                                    int64_t ldo, float* row_sumsq, int64_t sumsq_cols, void* vt, int64_t vt_col0,
                                    int64_t vt_ld, void* stream) {
  using namespace wanmi;
  clear_error();
  WANMI_REQUIRE(vt && ((uintptr_t)vt % 16) == 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm_qkv: vt must be a 16-byte aligned pointer");
  WANMI_REQUIRE(vt_col0 > 0 && vt_col0 < N && vt_col0 % TN == 0 && (N - vt_col0) % TN == 0, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm_qkv: vt_col0=%lld must be a multiple of %d inside (0, N)", (long long)vt_col0, TN);
  WANMI_REQUIRE(!row_sumsq || ((uintptr_t)row_sumsq % 4) == 0, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm_qkv: row_sumsq must be 4-byte aligned");
  WANMI_REQUIRE(sumsq_cols >= 0 && sumsq_cols <= vt_col0 && sumsq_cols % 128 == 0, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm_qkv: sumsq_cols=%lld must be a multiple of 128 in [0, vt_col0]", (long long)sumsq_cols);
  WANMI_REQUIRE(K % 32 == 0, WANMI_ERR_ARG, "wanmi_mxfp8_gemm_qkv: K=%lld must be a multiple of 32", (long long)K);
  // The V^T epilogue writes the token columns of the 256-token tiles it covers (zeros past M), so
  // padding past M is only written up to M rounded up to 256; with M == 0 nothing would be written.
  WANMI_REQUIRE(M > 0 && vt_ld <= (M + TM - 1) / TM * TM, WANMI_ERR_ARG,
                "wanmi_mxfp8_gemm_qkv: M=%lld must be positive and vt_ld=%lld at most M rounded up to %d",
                (long long)M, (long long)vt_ld, TM);
  // Q | K: the plain bf16 epilogue (with the Q partial sums) on the weight rows [0, vt_col0)
  int st = gemm_impl(a_codes, a_scales, w_codes, w_scales, row_scale, col_scale, bias, M, vt_col0, K, lda,
                     WANMI_EPI_BF16, out, ldo, nullptr, nullptr, nullptr, row_sumsq, row_sumsq ? sumsq_cols : 0,
                     vt_col0 / 128, nullptr, 0, stream);
  if (st != WANMI_OK) return st;
  // V: the weight rows [vt_col0, N), transposed accumulator, V^T epilogue
  return gemm_impl(a_codes, a_scales, w_codes + vt_col0 * K, w_scales + vt_col0 * (K / 32), row_scale,
                   col_scale ? col_scale + vt_col0 : nullptr, bias ? bias + vt_col0 : nullptr, M, N - vt_col0, K, lda,
                   kEpiVt, nullptr, 0, nullptr, nullptr, nullptr, nullptr, 0, 0, vt, vt_ld, stream);
}
