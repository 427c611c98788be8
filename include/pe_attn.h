/*
 * pe_attn.h — C ABI of the MI355X (gfx950) packed varlen attention library libpe_attn.so.
 *
 * Packed (padding-free) attention over flat [total_tokens, heads, head_dim] bf16 Q/K/V with
 * int32 cu_seqlens boundaries, the hot path of packed-encoders. Every entry point takes plain
 * pointers and sizes, never throws, and returns 0 or a negative PE_ATTN_E* status. Kernels are
 * launched on the caller's stream with no host synchronisation and no device-to-host reads,
 * so every entry point is safe inside HIP graph capture. The library allocates nothing: the
 * entry points that need scratch memory take a caller workspace, or (pe_varlen_attn_fwd_noalloc)
 * use a fixed array in device memory.
 *
 * Semantics (identical for every entry point):
 *   For each segment s with start = cu_seqlens[s], length L = cu_seqlens[s+1] - start, each
 *   query row i < L of query head h reads keys j < L of kv head h / (n_heads_q / n_heads_kv):
 *     allowed(i, j) = (window_left  < 0 || i - j <= window_left)
 *                  && (window_right < 0 || j - i <= window_right)
 *                  && (!causal || j <= i)
 *     out[i] = sum_j softmax_j(scale * q_i . k_j over allowed j) * v_j
 *   Arithmetic: fp32 scores and accumulation; probabilities are rounded to bf16 before the
 *   P.V product and the normaliser is an fp32 sum of the probabilities (of their bf16-rounded
 *   values in the head_dim-64 tiled kernel, of the unrounded ones elsewhere); the output is
 *   rounded to bf16. With a gate, out = bf16(bf16(out) * bf16(sigmoid(gate))).
 *   Rows at or beyond cu_seqlens[n_seq] are never written. Empty segments are allowed.
 *   Caller contract (not checked on device): cu_seqlens[0] = 0, non-decreasing,
 *   cu_seqlens[n_seq] <= total_tokens, and max_seqlen >= every segment length. The kernels'
 *   32-bit offsets are sized from max_seqlen, so a segment longer than it is skipped (its rows
 *   are left unwritten) rather than addressed.
 */
#ifndef PE_ATTN_H
#define PE_ATTN_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PE_ATTN_ABI_VERSION 9

#define PE_ATTN_OK 0
#define PE_ATTN_EINVAL (-1)       /* malformed arguments (maps to ValueError) */
#define PE_ATTN_EUNSUPPORTED (-2) /* well-formed but outside the kernels' envelope */
#define PE_ATTN_EWORKSPACE (-3)   /* workspace missing or too small */
#define PE_ATTN_ELAUNCH (-4)      /* a kernel launch failed (maps to RuntimeError) */
#define PE_ATTN_ESCRATCH (-5)     /* the call needs more than the library's static scratch */

#define PE_ATTN_DTYPE_BF16 1

typedef struct pe_attn_args {
    uint32_t struct_size; /* sizeof(pe_attn_args): guards against a mismatched header */
    int32_t dtype;        /* PE_ATTN_DTYPE_BF16 */
    const void *q;        /* [total_tokens, n_heads_q,  head_dim] */
    const void *k;        /* [total_tokens, n_heads_kv, head_dim] */
    const void *v;        /* [total_tokens, n_heads_kv, head_dim] */
    void *o;              /* [total_tokens, n_heads_q,  head_dim] (written); must not overlap q, k,
                             v, gate or the RoPE tables: workgroups write o while others still
                             read the inputs of their own rows' segment */
    const void *gate;     /* optional [total_tokens, n_heads_q, head_dim]; NULL for none */
    const int32_t *cu_seqlens; /* device [n_seq + 1] */
    /* strides in elements; the head_dim stride is 1. 16-byte alignment of every row is
       required: base pointers % 16 == 0 and token/head strides % 8 == 0. */
    int64_t q_stride_token, q_stride_head;
    int64_t k_stride_token, k_stride_head;
    int64_t v_stride_token, v_stride_head;
    int64_t o_stride_token, o_stride_head;
    int64_t gate_stride_token, gate_stride_head;
    int32_t n_seq;
    int32_t total_tokens;
    int32_t max_seqlen; /* host bound on every segment length */
    int32_t n_heads_q;
    int32_t n_heads_kv; /* divides n_heads_q */
    int32_t head_dim;   /* 64, 128 or 256 */
    float softmax_scale;
    int32_t window_left;  /* -1: unbounded */
    int32_t window_right; /* -1: unbounded */
    int32_t causal;       /* 0 or 1; causal is window_right = 0 */
    /* Per-segment routing: segments with length <= short_max run the LDS-resident short
       kernel, longer ones the tiled MFMA kernel. 0 sends every segment to the tiled kernel;
       -1 asks for the library's gfx950 default: max_seqlen (and max_seqlen_k) when it is at
       most 128 (every segment short), else 64 for head_dim 64 and 32 for head_dim 128. At most 128; head_dim 256 always runs the
       tiled kernel (the short kernel covers head_dim <= 128). */
    int32_t short_max;
    /* Query tiles (of 128 rows; 32 * 4 / gcd(GQA ratio, 4) rows with grouped heads) one
       workgroup of the tiled kernel walks in sequence, its key/value pipeline running across
       tile boundaries. 0 asks for the library's default; at most 64. */
    int32_t strip;
    /* Key/value segments distinct from the query segments (FlashAttention's cu_seqlens_k):
       device [n_seq + 1], or NULL for the query segments themselves (then the two fields
       below are ignored). k and v hold total_tokens_k rows. Query segment s is the TAIL of key
       segment s: its row r sits at key position r + (Lk - Lq), and the causal bound and the
       window are measured from there (the reference's prefixed form for rows continuing a
       shared prefix, packed_encoders/runtime/attention.py:15-19,236-245; flash_attn_varlen's
       bottom-right alignment). A row that reaches no key comes out as zero. Segments with both
       lengths <= short_max take the short kernel. */
    const int32_t *cu_seqlens_k;
    int32_t total_tokens_k;
    int32_t max_seqlen_k; /* host bound on every key segment length */
    /* Kernel for the long segments of a bounded band window each of whose rows spans five
       32-key blocks (ModernBERT's +-64: floor((31 + right) / 32) + ceil(left / 32) == 4), with
       head_dim 64, an odd GQA ratio and no cu_seqlens_k: 0 the library's choice (the streaming
       band kernel from 17667 query tiles of 128 rows x heads, the tiled kernel below), 1 the
       streaming band kernel, 2 the tiled kernel. Other calls ignore it. */
    int32_t band_kernel;
    /* Host lower bound on every query segment length, or 0 when not known (flash_attn's
       varlen interface carries max_seqlen only; a collator that packs host-known lengths
       knows both). When it exceeds the routing boundary no segment can take the short
       kernel: pe_attn_short_fwd launches nothing and the plan gives every segment to the
       tiled kernels, which serve any length, so a bound that is wrong costs time, never
       results. 0 <= min_seqlen <= max_seqlen. */
    int32_t min_seqlen;
    /* Fused RoPE prologue (the reference's apply_rope_bshd before its attention,
       packed_encoders/ops.py:485-499, _kernels/rope.py:302-349), or NULL for none. With
       tables, q and k are the projection's unrotated rows (typically strided views into the
       packed qkv) and the kernel applies split-half RoPE before the products: packed row r
       (query token r, key token r) takes row r % rope_table_rows of cos and sin [rows, head_dim]
       (bf16, rows rope_table_stride elements apart: per-token gathered tables, or the [S, D]
       tables of a dense [B, S] batch), with pe_rope_qkv_fwd's rounding, so the result is bit
       for bit that of pe_rope_qkv_fwd followed by the call on its q and k. Served by the short
       kernel: a call with tables needs head_dim 64 or 128, no cu_seqlens_k, and every segment
       within the routing boundary (max_seqlen <= the effective short_max), else
       PE_ATTN_EUNSUPPORTED. */
    const void *rope_cos;
    const void *rope_sin;
    int64_t rope_table_stride;
    int32_t rope_table_rows;
} pe_attn_args;

/* ABI version of the loaded library; callers compare it with PE_ATTN_ABI_VERSION. */
int pe_attn_abi_version(void);

/* Static text for a status code. */
const char *pe_attn_strerror(int status);

/* Bytes of device workspace pe_varlen_attn_fwd needs for these arguments (host-only, from
   n_seq, total_tokens, max_seqlen, min_seqlen, head geometry and short_max; never reads
   device memory). */
int pe_attn_workspace_size(const pe_attn_args *args, size_t *bytes);

/* Packed varlen attention, both kernels in one call. Segments are routed per segment on the
   device by their length (no host read of cu_seqlens): short ones to the LDS-resident kernel,
   long ones through a device-built, cost-ordered tile list to the tiled MFMA kernel.
   Replaces the reference's FlashAttention varlen leg (packed_encoders/ops.py:432-461,
   ops.py:521-532) and the varlen candidates of select_attention
   (packed_encoders/runtime/attention.py:66-126), GQA, causal, window and the fused sigmoid
   gate (packed_encoders/_kernels/hybrid.py:197-219) included. */
int pe_varlen_attn_fwd(const pe_attn_args *args, void *workspace, size_t workspace_bytes,
                       hipStream_t stream);

/* pe_varlen_attn_fwd with its workspace in a static device array of PE_ATTN_STATIC_SCRATCH_BYTES
   (one copy per GPU, held until the process ends) instead of a caller allocation: for callers
   that cannot allocate (code under HIP graph capture, tight serving loops, harnesses that
   forbid hipMalloc). No counterpart in the reference. It calls no allocating routine; its first
   call on a device looks the array's device address up once (hipGetSymbolAddress).
   Returns PE_ATTN_ESCRATCH, launching nothing, when pe_attn_workspace_size exceeds the array
   (at 1 MiB: about 65,000 (segment, query tile) entries). Every call on one GPU shares that
   GPU's array: calls that overlap on one GPU (other streams, other threads) race and must be
   serialised by the caller. */
#define PE_ATTN_STATIC_SCRATCH_BYTES (1u << 20)
int pe_varlen_attn_fwd_noalloc(const pe_attn_args *args, hipStream_t stream);

/* The three stages pe_varlen_attn_fwd runs, for callers that reuse one plan across calls
   (the 22 layers of a packed forward share cu_seqlens: one plan per window kind serves all
   of them) or time one kernel. A plan is valid for arguments with the same cu_seqlens
   contents, n_seq, total_tokens, max_seqlen, min_seqlen, head counts, window, causal and
   short_max.
   pe_attn_plan: build the cost-ordered (segment, query tile) list of the tiled kernel into
     the workspace (no-op when no segment can exceed short_max). The workspace starts with two
     int32 words: the entries written and the entries needed. They differ only when the
     arguments break the caller contract that sized the list (cu_seqlens decreasing or past
     total_tokens); segments longer than max_seqlen (keys: max_seqlen_k) take no entry.
   pe_attn_short_fwd: the short kernel over segments with length <= short_max (no-op for 0).
   pe_attn_tiled_fwd: the tiled kernel over a planned workspace. */
int pe_attn_plan(const pe_attn_args *args, void *workspace, size_t workspace_bytes, hipStream_t stream);
int pe_attn_short_fwd(const pe_attn_args *args, hipStream_t stream);
int pe_attn_tiled_fwd(const pe_attn_args *args, const void *workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* Packed short attention: every segment through the LDS-resident short kernel. Requires
   0 < max_seqlen <= 128 and head_dim <= 128; short_max is ignored. Needs no workspace.
   Replaces packed_short_attention / _launch_packed_short_attention
   (packed_encoders/_kernels/triton_packed_attention.py:175-236). */
int pe_packed_short_attn_fwd(const pe_attn_args *args, hipStream_t stream);

/* The short kernel's static launch choice for a max_seqlen (no runtime autotuning):
   out[0] = query rows per wave (block_m), out[1] = key capacity held in LDS,
   out[2] = heads per workgroup, out[3] = waves per workgroup.
   Replaces select_packed_short_attention_config
   (packed_encoders/_kernels/triton_packed_attention.py:29-42). */
int pe_attn_short_config(int32_t max_seqlen, int32_t head_dim, int32_t out[4]);

/* The kernels pe_varlen_attn_fwd runs for these arguments (host-only, like the workspace
   size): out[0] the short kernel's key capacity (0: no short kernel), out[1] the long-segment
   kernel (PE_ATTN_KERNEL_*), out[2] its query tiles per workgroup (strip), out[3] its query
   rows per tile, out[4] the short kernel's query heads per workgroup (fewer than
   pe_attn_short_config's when the batch would leave CUs idle) and out[5] its workgroups.
   No counterpart in the reference; for profiling and tests. */
#define PE_ATTN_KERNEL_NONE 0
#define PE_ATTN_KERNEL_TILED 1    /* tiled_attn_kernel: head_dim 64 windowed or causal */
#define PE_ATTN_KERNEL_GLOBAL64 2 /* global64_attn_kernel: head_dim 64 unbounded */
#define PE_ATTN_KERNEL_BAND64 3   /* band64_attn_kernel: head_dim 64 streaming band */
#define PE_ATTN_KERNEL_WIDE 4     /* wide_attn_kernel: head_dim 128 */
#define PE_ATTN_KERNEL_WIDE16 5   /* wide16_attn_kernel: head_dim 256 */
int pe_attn_kernels(const pe_attn_args *args, int32_t out[6]);

/* Split-half rotary embedding straight from the packed QKV projection: the producer of the
   layout the attention entry points read (q, k contiguous [n_rows, n_heads, head_dim]; v stays
   a strided view of qkv). Row r of qkv [n_rows, 3 * n_heads * head_dim] (q at column 0, k at
   n_heads * head_dim) uses row r % table_rows of the cos / sin tables [table_rows, head_dim]:
   per-token gathered tables for a packed batch, [S, head_dim] tables for a dense [B, S] one.
     q_out[r, h, i]       = bf16(q[i] * cos[i] - q[i + D/2] * sin[i])
     q_out[r, h, i + D/2] = bf16(q[i + D/2] * cos[i + D/2] + q[i] * sin[i + D/2])   (i < D/2)
   in fp32 with each product rounded before the sum; k likewise. 16-byte alignment of every
   row is required (pointers % 16 == 0, strides % 8 == 0). */
typedef struct pe_rope_args {
    uint32_t struct_size; /* sizeof(pe_rope_args) */
    int32_t dtype;        /* PE_ATTN_DTYPE_BF16 */
    const void *qkv;      /* [n_rows, 3 * n_heads * head_dim], row stride qkv_stride_row */
    const void *cos;      /* [table_rows, head_dim], row stride table_stride_row */
    const void *sin;      /* same shape and stride as cos */
    void *q_out;          /* [n_rows, n_heads, head_dim] contiguous (written) */
    void *k_out;          /* [n_rows, n_heads, head_dim] contiguous (written) */
    int64_t qkv_stride_row;   /* elements */
    int64_t table_stride_row; /* elements */
    int32_t table_rows;
    int32_t n_rows;
    int32_t n_heads;
    int32_t head_dim; /* 64, 128 or 256 */
} pe_rope_args;

/* Replaces apply_rope_bshd (packed_encoders/_kernels/rope.py:302-349) on the packed attention
   path (packed_encoders/ops.py:464-499). */
int pe_rope_qkv_fwd(const pe_rope_args *args, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PE_ATTN_H */
