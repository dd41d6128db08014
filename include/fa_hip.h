/*
 * fa_hip.h -- C ABI of the MI355X (gfx950) FlashAttention-2 forward.
 *
 *   O = softmax(Q K^T * softmax_scale) V      Q, K, V, O: [B, H, N, D] fp16, contiguous
 *
 * Plain C: pointers, fixed-width integers and a void* stream. No PyTorch or C++ types, so the
 * library can be bound from ctypes, a PyTorch extension or any C caller.
 *
 * Replaces, one for one, the torch-free C++ API of the reference:
 *   fa_params          <- fa::FlashFwdParams + fa::Variant   (csrc/flash_fwd.h:12-30)
 *   fa_flash_fwd       <- void fa::flash_fwd(const FlashFwdParams&, cudaStream_t)
 *                                                            (csrc/flash_fwd.h:33,
 *                                                             csrc/kernels/flash_fwd.cu:625-652)
 *   fa_last_error      <- the what() text of the std::invalid_argument / std::runtime_error the
 *                         reference throws (csrc/kernels/flash_fwd.cu:626-651, csrc/common.cuh:15-26)
 * The reference signals errors with C++ exceptions; a C ABI cannot, so every entry point
 * returns an fa_status and keeps the message in a thread-local buffer.
 */
#ifndef FA_HIP_H_
#define FA_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes. FA_EINVAL plays the role of std::invalid_argument, FA_EHIP of the
 * std::runtime_error that CUDA_CHECK raises (csrc/common.cuh:15-26). */
typedef enum fa_status {
    FA_OK = 0,
    FA_EINVAL = 1, /* bad argument: nothing was launched                                     */
    FA_EHIP = 2    /* the HIP runtime refused the launch (launch-configuration error)        */
} fa_status;

/* Kernel build selector; same values as fa::Variant (csrc/flash_fwd.h:12-16).
 * On CDNA4 the f16 MFMA always accumulates in fp32 and has no faster fp16-accumulate form,
 * so FA_VARIANT_FP16ACC runs the same kernel as FA_VARIANT_OPT (bitwise identical output). */
typedef enum fa_variant {
    FA_VARIANT_BASELINE = 0, /* first correct MI355X kernel: exact rescaling, smaller tiles   */
    FA_VARIANT_OPT = 1,      /* tuned kernel (default)                                        */
    FA_VARIANT_FP16ACC = 2   /* accepted for API parity; identical to FA_VARIANT_OPT         */
} fa_variant;

/* Mirrors fa::FlashFwdParams (csrc/flash_fwd.h:18-30) with fixed-width fields. */
typedef struct fa_params {
    const void* q;         /* [B, H, N, D] fp16, contiguous, 16-byte aligned                   */
    const void* k;         /* [B, H, N, D] fp16, contiguous, 16-byte aligned                   */
    const void* v;         /* [B, H, N, D] fp16, contiguous, 16-byte aligned                   */
    void* o;               /* [B, H, N, D] fp16, contiguous, 16-byte aligned (output)          */
    int32_t batch;         /* B > 0                                                            */
    int32_t heads;         /* H > 0                                                            */
    int32_t seqlen;        /* N > 0, same for queries and keys                                 */
    int32_t head_dim;      /* D: 64 or 128                                                     */
    float softmax_scale;   /* usually 1/sqrt(D); any finite value                              */
    uint8_t causal;        /* 0 or 1: key j is visible to query i iff j <= i                   */
    uint8_t variant;       /* an fa_variant value                                              */
    uint8_t reserved[2];   /* must be zero                                                     */
} fa_params;

/* Launches the forward kernel asynchronously on `stream` (a hipStream_t; NULL = the null
 * stream) on the current HIP device and returns without synchronizing. All argument checks
 * run before any HIP call, so FA_EINVAL never touches the device. Writes only rows < N of o.
 * Allocates nothing per call; re-entrant. (The library's code object holds the 64 MiB scratch
 * array of fa_flash_fwd_splitkv_static below, FA_STATIC_SCRATCH_BYTES, so a process that
 * launches any of its kernels on a GPU holds that much device memory there until it ends.)
 * Faults during execution surface at the caller's next synchronization, as with any
 * asynchronous HIP launch.
 * Replaces fa::flash_fwd (csrc/flash_fwd.h:33; checks at csrc/kernels/flash_fwd.cu:626-651). */
int fa_flash_fwd(const fa_params* params, void* stream);

/* Message of the last failing call on this thread ("" after a success). The pointer stays
 * valid until the next fa_* call on the same thread. */
const char* fa_last_error(void);

/* fa_flash_fwd that also writes the log-sum-exp of every row:
 *   lse[b, h, i] = log(sum_j exp(softmax_scale * q_i . k_j))   (natural log, over visible keys)
 * lse: [B, H, N] fp32, contiguous, 4-byte aligned. O is bitwise the output of fa_flash_fwd.
 * The LSE is what merging partial attention results needs (split-KV below, sequence/context
 * parallelism across GPUs) and what a backward pass recomputes P from. No counterpart in the
 * reference, whose epilogue keeps only O (csrc/kernels/flash_fwd.cu:526-560). */
int fa_flash_fwd_lse(const fa_params* params, float* lse, void* stream);

/* Split-KV ("flash-decoding" style) forward for grids too small to fill the GPU (few heads,
 * long sequences): the key tiles of every query block are cut into ranges, one workgroup per
 * (query block, range) writes a partial O and LSE per row to the caller's workspace, and a
 * second kernel merges them by their LSEs. Same results as fa_flash_fwd within fp32 rounding
 * of the merge (not bitwise). No counterpart in the reference (its docs list split-KV as not
 * done: docs/optimizations.md:372-373).
 * fa_splitkv_plan reports the ranges and the workspace size for num_splits (0 = automatic:
 * 256 to 1024 workgroups with work, by head_dim and causal), and whether the split path is the
 * faster one for these params; host-only. fa_flash_fwd_splitkv runs it: lse may be NULL;
 * workspace must be 16-byte aligned and hold at least workspace_bytes of the plan for the same
 * params and num_splits. Two launches on `stream`; allocates nothing. The variant field is
 * checked but every variant runs the same split tile. */
typedef struct fa_splitkv_info {
    int32_t num_splits;       /* key ranges per query block (ranges past a causal block's last
                                 key tile are skipped)                                        */
    int32_t tiles_per_split;  /* key tiles per range                                          */
    int32_t block_q;          /* query rows per workgroup of the partial pass                 */
    int32_t block_k;          /* keys per tile                                                */
    uint64_t workspace_bytes; /* num_splits * B * H * N * (D + 1) * 4                         */
    int32_t preferred;        /* 1 if the automatic split-KV plan is expected to beat
                                 fa_flash_fwd on these params (variant not baseline, a grid
                                 that leaves most CUs idle, N >= 4096; causal at D = 64:
                                 N >= 16384; or a causal grid of 256 to 288 query blocks of
                                 256 rows, N >= 8192, where the automatic plan takes two
                                 ranges at D = 128), else 0; independent of num_splits. The PyTorch
                                 binding's forward takes the split path exactly when it is 1. */
    int32_t reserved;         /* 0                                                            */
} fa_splitkv_info;
int fa_splitkv_plan(const fa_params* params, int32_t num_splits, fa_splitkv_info* out);

/* Head split of a non-causal call whose grid of one-workgroup-per-CU items leaves its last round
 * mostly empty (no counterpart in the reference): *single_heads = h > 0 means that the first h
 * of the B*H heads (flattened [B*H, N, D]) are best run by fa_flash_fwd (batch 1, heads h: whole
 * rounds of workgroups) and the other B*H - h by fa_flash_fwd_splitkv (pointers advanced by
 * h*N*D elements, LSE by h*N); 0 means one fa_flash_fwd call. The PyTorch binding's forward and
 * forward_lse follow it. Same argument checks as fa_splitkv_plan; host-only. */
int fa_tail_plan(const fa_params* params, int64_t* single_heads);
int fa_flash_fwd_splitkv(const fa_params* params, float* lse, int32_t num_splits,
                         void* workspace, uint64_t workspace_bytes, void* stream);

/* fa_flash_fwd_splitkv without a workspace argument and without any allocation: the partial
 * results go to a static scratch array of FA_STATIC_SCRATCH_BYTES (64 MiB) that the library
 * holds on every GPU it runs on until the process ends (its device address is looked up once
 * per device, on the first call with that device current). For callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc. No counterpart in the reference. Same arguments, checks and results (bitwise) as
 * fa_flash_fwd_splitkv with the same num_splits; returns FA_EINVAL, launching nothing, when the
 * plan's workspace_bytes exceeds the scratch (pass a smaller num_splits then). Every call on a
 * GPU shares that GPU's scratch: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialized by the caller. The current HIP device must be the device of
 * `stream`. */
#define FA_STATIC_SCRATCH_BYTES (64ULL << 20)
int fa_flash_fwd_splitkv_static(const fa_params* params, float* lse, int32_t num_splits,
                                void* stream);

/* Main-loop schedule of a tile (fa_tile_info.schedule). */
typedef enum fa_schedule {
    FA_SCHED_SIMPLE = 0,     /* each wave runs S = QK^T, softmax and O += PV of a tile in turn,
                                on 32x32x16 MFMAs                                             */
    FA_SCHED_KSPLIT = 3,     /* small grids: two waves per 32 query rows, each on every second
                                key tile, merged through LDS                                  */
    FA_SCHED_PINGPONG16 = 4, /* two groups of waves alternate between an MFMA-only phase and a
                                softmax phase, on 16x16x32 MFMAs                               */
    FA_SCHED_KSPLIT4 = 5,    /* tiny grids: four waves per 32 query rows                       */
    FA_SCHED_SIMPLE16 = 6    /* the simple schedule on 16x16x32 MFMAs                          */
} fa_schedule;

/* Tile geometry fa_flash_fwd launches for these parameters: query rows per workgroup, keys per
 * tile, wavefronts per workgroup, LDS bytes per workgroup and the main-loop schedule. The
 * choice depends on variant, head_dim, causal, seqlen and batch * heads (small grids get
 * smaller workgroups); the four pointers are not read. Host-only, touches no device. No
 * counterpart function in the reference, whose tiles are compile-time `using` lines
 * (csrc/kernels/flash_fwd.cu:597-612); exported so that tests and the benchmark can report and
 * check the grid the kernel runs. */
typedef struct fa_tile_info {
    int32_t block_q;       /* BR: query rows per workgroup                                     */
    int32_t block_k;       /* BC: key rows per K/V tile                                        */
    int32_t waves;         /* wavefronts (64 lanes) per workgroup                              */
    int32_t lds_bytes;     /* LDS per workgroup                                                */
    int32_t schedule;      /* an fa_schedule value                                             */
} fa_tile_info;
int fa_tile_config(const fa_params* params, fa_tile_info* out);

/* Library version string and softmax build options, e.g.
 * "fa_hip 0.2.0 gfx950 pp16_unchecked=1 pp16_margin=0 pp16_spread=9". */
const char* fa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_HIP_H_ */
