// Internal launcher API between the C-ABI host layer and the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ribn_amd {

// Members one wave-GEMV launch serves (weights read once for all of them);
// larger batches are split by the host into launch groups. K above one slice
// (4096) takes two members per launch.
constexpr int kWaveMaxMembers = 8;
// Weights one grouped wave-GEMV launch streams (they share one activation vector).
constexpr int kMaxGroup = 4;
// LDS the wave GEMV may use for its quantized [members][K] activation
// records, and the largest K its staging covers.
constexpr long long kWaveMaxLdsBytes = 128 * 1024;
constexpr int kWaveMaxK = 16384;
// K one wave covers per unit (16 super-blocks); the many-member and gate/up
// pair forms need K within it.
constexpr int kSliceK = 4096;
// Largest K of the f32 GEMV's slice-split form, which stages one slice per
// workgroup and so serves a K beyond kWaveMaxK (plain and accumulating
// products, no fused prologue), and the bytes of slice totals it may keep
// in the context scratch.
constexpr int kF32SplitMaxK = 65536;
constexpr size_t kF32SplitScratchBytes = (size_t)2 << 20;

// Activation prologue of the wave GEMV: plain x, RMSNorm(x; gamma), or
// SwiGLU silu(x) * x2.
constexpr int kProPlain = 0;
constexpr int kProNorm = 1;
constexpr int kProSwiglu = 2;
// Members one SwiGLU-prologue launch serves (the host splits larger batches).
constexpr int kSwigluMaxMembers = 2;

// A residual update the f32-faithful matrix-core GEMV left pending: the raw
// split sums of an accumulating product, y[m][r] += sum over splits in split
// order of partial[split][m][r] (what f32mma_reduce_kernel would have added).
// The next f32-faithful call whose input x is that y adds them first
// (identical bits) and stores y, so the reduce launch disappears.
struct F32MmaFold {
    float* y;              // [members][rows]
    const float* partial;  // [splits][members][rows]
    int splits;            // 0: nothing pending
    int members;
    int rows;
};

struct WaveGemvArgs {
    const uint8_t* w[kMaxGroup];
    uint32_t wbytes[kMaxGroup];
    float* y[kMaxGroup];      // y[i] is [members][N_i]
    int rows_end[kMaxGroup];  // prefix sums of N_i
    int count;
    int total_rows;
    const float* x;           // [members][K]
    const float* gamma;       // RMSNorm weight [K], or null for a plain GEMV
    const float* x2;          // SwiGLU: the up projection [members][K] (x is the gate), or null
    float eps;
    int K;
    int members;
    int accumulate;           // nonzero: y += W x' (fused residual add) instead of y = W x'
    // nonzero: w[0] / w[1] are gate / up of equal shape, and y[0] [members][N]
    // receives silu(gate . x') * (up . x') (K <= 4096; y[1] unused)
    int pair_swiglu;
    // Arithmetic: kArithF32 (f32 activations, the default) or kArithFixed16
    // (block fixed-point activations with integer dot products, opt-in).
    int arith;
    // f32 launches split by slice: [slices][members][total_rows] slice totals
    float* partial;
    // f32-faithful matrix-core path only (9..64 members): `defer` (an
    // accumulating single-weight product) receives its pending split sums
    // instead of a reduce launch, or splits = 0 if it finished; `fold` (an
    // input x equal to fold->y) adds pending sums into x first.
    F32MmaFold* defer;
    const F32MmaFold* fold;
};

constexpr int kArithF32 = 0;
constexpr int kArithFixed16 = 1;

// Largest member count one f32 wave-GEMV launch stages for this K (0 if none).
int f32_max_members(int K);
// The f32-activation wave GEMV (gemv_f32.hip); members <= f32_max_members(K).
hipError_t launch_gemv_f32(int value_type, const WaveGemvArgs& args, int cu_count, hipStream_t stream);
// Its slice-split form over K spanning several slices (plain prologue, no
// pairs): 3..8 members up to kWaveMaxK, 1..8 members beyond it (up to
// kF32SplitMaxK); args.partial holds f32_split_partial_bytes of slice totals,
// which a second launch adds in slice order into y.
size_t f32_split_partial_bytes(int members, int K, int total_rows);
hipError_t launch_gemv_f32_split(int value_type, const WaveGemvArgs& args, int cu_count, hipStream_t stream);
// Members per slice-split launch for a K beyond kWaveMaxK (0: that form does
// not serve this shape, whose slice totals would not fit the scratch).
int f32_long_k_members(int K, int total_rows);

// Largest member count one wave launch can stage for this K (0 if none).
int wave_max_members(int K);

// ---- batched GEMV on the int8 matrix cores (gemv_mfma.hip), up to 16 members

constexpr int kMfmaMaxMembers = 16;
// From this many members the matrix cores beat the wave GEMV (measured on
// MI355X over the Qwen3-8B projections); a K spanning several slices, where
// the wave GEMV takes two members per launch, from kMfmaMinMembersLongK.
constexpr int kMfmaMinMembers = 5;
constexpr int kMfmaMinMembersLongK = 4;

// Byte offsets of the packed activations of `members` x K (K a multiple of
// 256): MFMA fragments, per-group minimum-term inputs, per-block unscales and
// per-workgroup partial sums of squares.
struct Act16Layout {
    uint32_t frag, mina, ublk, ssq, total;
    int nb;     // super-blocks of K
    int parts;  // pack workgroups per member (partial sums of squares)
    int hl;     // up to 8 members: each fragment holds high digits in rows 0-7, low digits in rows 8-15
};
Act16Layout act16_layout(int members, int K);

struct MfmaGemvArgs {
    const uint8_t* w[kMaxGroup];
    uint32_t wbytes[kMaxGroup];
    float* y[kMaxGroup];      // y[i] is [members][N_i]
    int rows_end[kMaxGroup];  // prefix sums of N_i; all but the last a multiple of 16
    int count;
    int total_rows;
    const void* act;          // launch_pack_act16 output for these members and K
    uint32_t act_bytes;
    Act16Layout L;
    int K;
    int members;
    int has_norm;             // the activations were packed with gamma: outputs are divided by rms(x)
    float eps;
    int accumulate;           // nonzero: y += W x'
    int pair_swiglu;          // w[0] / w[1] gate / up of equal shape; y[0] receives silu(g) * u
};

bool gemv_mfma_supported(int value_type);
// Packs x [members][K] (times gamma when given) for launch_gemv_mfma.
hipError_t launch_pack_act16(const float* x, const float* gamma, int members, int K, void* act,
                             hipStream_t stream);
hipError_t launch_gemv_mfma(int value_type, const MfmaGemvArgs& args, int cu_count, hipStream_t stream);

// ---- f32-faithful batched GEMV on the matrix cores (gemv_f32mma.hip)
//
// The default f32 arithmetic for 9..64 members: exact products on the
// matrix cores (Q4_K / Q5_K: quants times group scale exact in f16 against
// activations in two f16 pieces; Q6_K: quants exact in bf16 against three
// bf16 pieces), f32 accumulation, so results agree with the f32 wave GEMV to
// f32 rounding (not bit for bit); the weights are read once for the whole
// batch. Up to 8 members stay on the wave GEMV, whose rows are bit-identical
// to the single-member call.
constexpr int kF32MmaMinMembers = 9;
constexpr int kF32MmaMaxMembers = 64;
// Byte offsets of the packed activations of `members` x K (K a multiple of
// 256): the pieces' MFMA fragments, f32 group sums, inverse block scales (f16
// form), per-workgroup partial sums of squares.
struct F32MmaLayout {
    uint32_t frag, xsum, iscale, ssq, total;
    int nb;     // super-blocks of K
    int tiles;  // member tiles of 16
    int parts;  // pack workgroups per member
};
// pieces: 3 (bf16 pieces, Q6_K) or 2 (f16 pieces, Q4_K / Q5_K); 3 sizes both.
F32MmaLayout f32mma_layout(int members, int K, int pieces = 3);
// Whether launch_gemv_f32mma serves this call (type, 9..64 members, K, pairs
// of whole tiles, not both RMSNorm and SwiGLU prologues).
bool f32mma_supported(int value_type, const WaveGemvArgs& args);
// Split-K partial room a context keeps after the packed activations.
constexpr size_t kF32MmaPartialBytes = (size_t)16 << 20;
// Pack (RMSNorm or SwiGLU prologue fused) + product (+ an ordered split-K
// reduce when the row groups alone do not fill the CUs); `scratch` holds
// f32mma_layout(members, K).total bytes, then the partials.
hipError_t launch_gemv_f32mma(int value_type, const WaveGemvArgs& args, void* scratch, size_t scratch_bytes,
                              int cu_count, hipStream_t stream);
// Adds a pending F32MmaFold into its y on its own (when no f32-faithful call
// consumes it) and clears it; nothing when none is pending.
hipError_t launch_f32mma_fold_flush(F32MmaFold* fold, hipStream_t stream);

// ---- Q8_1 activations and the integer-dot GEMV (q8_1.hip)

constexpr int kQ8MaxMembers = 8;
// Packs `blocks` 32-value blocks of x into nine words each.
hipError_t launch_quantize_q8_1(const float* x, uint32_t* out, uint32_t blocks, hipStream_t stream);
// y [members][N] from Q8_1-packed x [members][K / 32][9] (members <= kQ8MaxMembers).
hipError_t launch_gemv_q8_1(int value_type, const uint8_t* w, uint32_t wbytes, const uint32_t* x, float* y, int K,
                            int N, int members, hipStream_t stream);

// ---- GEMV dispatch used by the C ABI and the decoder

// Device scratch (bytes) a context reserves for launch_gemv's packed activations.
size_t gemv_act_scratch_bytes();
// Members one launch_gemv call may carry for this shape and arithmetic.
int gemv_launch_members(int value_type, int K, bool swiglu_prologue, int arith);
// kArithF32: 9..64 members on the matrix cores (launch_gemv_f32mma),
// else the f32 wave GEMV, split into the launch groups it stages.
// kArithFixed16: the block fixed-point wave GEMV, or from kMfmaMinMembers
// (kMfmaMinMembersLongK for K spanning several slices) up to 16 members
// without the SwiGLU prologue, packed activations through the matrix-core
// GEMV (two launches).
hipError_t launch_gemv(int value_type, const WaveGemvArgs& args, void* act_scratch, int cu_count,
                       hipStream_t stream);

hipError_t launch_dequant(int value_type, const uint8_t* w, uint32_t wbytes, float* out, uint32_t nblocks,
                          hipStream_t stream);

hipError_t launch_gemv_exact(int value_type, const uint8_t* w, uint32_t wbytes, const float* x, float* y,
                             int K, int N, int members, hipStream_t stream);

// args.gamma != nullptr: RMSNorm(x; gamma, eps) is fused into the activation
// load; args.x2 != nullptr: the activation is silu(x) * x2 (members <= 2, no
// gamma); args.accumulate: outputs are added into y; args.pair_swiglu: the
// gate/up pair epilogue (see WaveGemvArgs).
hipError_t launch_gemv_wave(int value_type, const WaveGemvArgs& args, int cu_count, hipStream_t stream);

// Gathers and dequantises rows of a [hidden, vocab] table: tokens[m] (device
// array) or `token` when tokens is null; out is [members][hidden].
hipError_t launch_embedding(int value_type, const uint8_t* w, uint32_t wbytes, const uint32_t* tokens,
                            uint32_t token, float* out, uint32_t blocks_per_token, uint32_t vocab, uint32_t members,
                            hipStream_t stream);

// Prefill / large-batch matmul (qgemm.hip). The activations pass through an
// f16 workspace of gemm_workspace_bytes(M, K) bytes: launch_act_f16 fills it
// (optionally RMSNorm-fused), launch_qgemm consumes it.
constexpr int kGemmMaxK = 16384;
// The workspace layout covers the activations and up to eight split-K partial
// [tokens][N] tiles; launch_qgemm splits K only as far as the space reserved.
size_t gemm_workspace_bytes(size_t tokens, size_t K, size_t N);
hipError_t launch_act_f16(bool bf16_in, const void* x, const float* gamma, float eps, int M, int K, void* workspace,
                          hipStream_t stream);
hipError_t launch_qgemm(int value_type, const uint8_t* w, uint32_t wbytes, void* workspace, size_t workspace_bytes,
                        float* y, int M, int N, int K, int cu_count, hipStream_t stream);
// Activation stages of the decoder's prompt prefill (f32 [M][K], K a multiple
// of 8): x += r (stored back to x), then RMSNorm with gamma, into the f16
// workspace; or silu(gate) * up into it.
hipError_t launch_act_f16_residual(float* x, const float* r, const float* gamma, float eps, int M, int K,
                                   void* workspace, hipStream_t stream);
hipError_t launch_act_f16_swiglu(const float* gate, const float* up, int M, int K, void* workspace,
                                 hipStream_t stream);

hipError_t launch_rms_norm(const float* x, const float* w, float* y, int length, int members, float eps,
                           hipStream_t stream);

}  // namespace ribn_amd
