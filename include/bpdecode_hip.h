/*
 * bpdecode_hip.h -- C ABI of libbpdecode_hip.so, the MI355X (gfx950) library
 * behind bpdecode_amd's batched constraint step.
 *
 * Plain pointers and sizes only.  Every entry point returns BPD_OK (0) or an
 * error code; bpd_last_error() then describes the failure (thread-local).
 * The two that return a value on success (bpd_pda_feed, a verdict;
 * bpd_host_frame_lists, a count) return their error codes negated.
 * Device entry points take device pointers and a hipStream_t (as void*),
 * enqueue work on that stream and return without synchronising.  Host entry
 * points (bpd_host_*) take host pointers and run on the calling thread; they
 * serve the CPU-tensor side of the same operator set.  The library allocates
 * no device memory: buffers an operation needs beyond its inputs and outputs
 * are passed in as a workspace whose size the matching *_workspace_bytes
 * function reports.
 *
 * Layouts (identical to the reference's tensor bundles):
 *   tok_next  int32 [num_states, vocab] row-major; -1 = token rejected.
 *   states    int32 pool; FREE = -2, BROKEN = -1.  With `slots` non-NULL the
 *             state of row b is states[slots[b]] (slots int64), otherwise
 *             states[b].
 *   pending   int64 [2 * num_pending]: queued pool writes (num_pending
 *             distinct slots, then their values).  An entry point that takes
 *             them applies them before it reads the pool: a row whose slot
 *             is queued reads the queued value, and every queued value is
 *             stored into the pool by the same launch.
 *   logits    [rows, ld] elements of `dtype`, unit column stride.
 *   configs   int32 [*, BPD_PDA_CONFIG_WORDS] = {num_configs, saturated,
 *             depth[8], stack[8][32]} (padding-free PdaConfigSet).
 *   bits      uint32 [rows, ceil(vocab/32)], LSB-first.
 */
#ifndef BPDECODE_HIP_H_
#define BPDECODE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BPD_OK 0
#define BPD_ERR_INVALID 1     /* bad argument: shape, dtype, range, alignment */
#define BPD_ERR_HIP 2         /* HIP runtime / launch failure */
#define BPD_ERR_OVERFLOW 3    /* fill value not representable in the logits dtype */
#define BPD_ERR_UNSUPPORTED 4 /* table too large for a kernel's encoding */

#define BPD_DTYPE_F32 0
#define BPD_DTYPE_F16 1
#define BPD_DTYPE_BF16 2
#define BPD_DTYPE_F64 3 /* dense tok_next mask only (bpd_dense_apply_mask*) */

#define BPD_INDEX_I32 0
#define BPD_INDEX_I64 1
#define BPD_INDEX_I64_LOW32 2 /* int64 ids read as their low 32 bits, as tensor.to(torch.int32) */

/* Queued state-pool writes a dense mask or commit launch applies itself. */
#define BPD_MAX_FUSED_PENDING 256

/* Bits OR-ed into the optional `err` word by kernels (device int32). */
#define BPD_FLAG_STATE_RANGE 1 /* a state >= num_states was read */
#define BPD_FLAG_TOKEN_RANGE 2 /* a token outside [-vocab, vocab) was read */

#define BPD_PDA_MAX_CONFIGS 8
#define BPD_PDA_MAX_DEPTH 32
#define BPD_PDA_CONFIG_WORDS (2 + BPD_PDA_MAX_CONFIGS + BPD_PDA_MAX_CONFIGS * BPD_PDA_MAX_DEPTH)

#define BPD_PDA_EDGE_EPS 0
#define BPD_PDA_EDGE_BYTE 1
#define BPD_PDA_EDGE_CALL 2

const char* bpd_last_error(void);
int bpd_abi_version(void);

/* ---------------------------------------------------------------- dense --
 * bpd_dense_apply_mask: logits[b, t] = neg_inf (converted to dtype as ATen's
 * checked scalar conversion does) iff state(b) < 0 or
 * tok_next[state(b), t] == -1; other entries are left bit-identical (never
 * read or written).  dtype: float32, float16, bfloat16 or float64; logits
 * need only element alignment.  A state >= num_states masks the row and sets
 * BPD_FLAG_STATE_RANGE in `err`.  Queued pool writes (`pending`, at most
 * BPD_MAX_FUSED_PENDING) are applied first.
 * Replaces the tok_next branch of ops.apply_mask_ (ops.py:271-276), which
 * ConstraintBatch.apply_mask (batch.py:176-190) calls after gathering
 * states = _state[slots]; the gather is fused here via `slots`.
 */
int bpd_dense_apply_mask(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                         const int32_t* tok_next, int32_t num_states, int32_t* states,
                         const int64_t* slots, const int64_t* pending, int64_t num_pending,
                         double neg_inf, int32_t* err, void* stream);

/* bpd_dense_apply_mask_bits: the same mask from the packed allow-bit table
 * (uint32 [num_states, words], words = ceil(vocab/32), bit t of row s set iff
 * tok_next[s, t] != -1 -- bpd_dense_compute_mask over every state builds it).
 * Results are identical to bpd_dense_apply_mask; the table read per row is
 * vocab/8 bytes instead of 4*vocab.  Serves the same reference entry points
 * (ops.py:271-276 via batch.py:176-190). */
int bpd_dense_apply_mask_bits(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                              const uint32_t* allow_bits, int64_t words, int32_t num_states,
                              int32_t* states, const int64_t* slots, const int64_t* pending,
                              int64_t num_pending, double neg_inf, int32_t* err, void* stream);

/* bpd_dense_advance: nxt = state(b) < 0 ? -1 : tok_next[state(b), t(b)], where
 * t(b) is tokens[b] read per token_dtype (BPD_INDEX_I32, BPD_INDEX_I64, or
 * BPD_INDEX_I64_LOW32 for the int32 cast ConstraintBatch.commit applies,
 * batch.py:213) and a negative t indexes from the end as torch advanced
 * indexing does; an id out of [-vocab, vocab) yields -1 and sets
 * BPD_FLAG_TOKEN_RANGE.  Writes next_out[b] (if non-NULL) and, with
 * write_back, stores nxt into the pool slot it was read from; all reads
 * happen before any write-back.  Queued pool writes (`pending`, needs
 * write_back and rows <= 4096) are applied first.  Replaces
 * ops.advance_state's tok_next branch (ops.py:301-306) plus
 * ConstraintBatch.commit's scatter (batch.py:206-215).
 */
int bpd_dense_advance(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                      int32_t* states, const int64_t* slots, const int64_t* pending,
                      int64_t num_pending, const void* tokens, int token_dtype, int64_t rows,
                      int32_t* next_out, int write_back, int32_t* err, void* stream);

/* bpd_dense_compute_mask: packed allow bits from tok_next (bit t of row b set
 * iff state(b) >= 0 and tok_next[state(b), t] != -1).  Dense counterpart of
 * compute_mask_batch (mask.hpp:55-57, torch_ops.cpp:154-189). */
int bpd_dense_compute_mask(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                           const int32_t* states, const int64_t* slots, int64_t rows,
                           uint32_t* bits, int32_t* err, void* stream);

/* bpd_build_tok_next: the dense table of build_token_transitions
 * (ops.py:143-197) on the device: tok_next[r, t] = walk of token t's symbol
 * classes from row_states[r] (every state 0..num_states-1 when row_states is
 * NULL), -1 on reaching `dead` or ending in a non-live state; the EOS column
 * is s for an accepting s and -1 otherwise. */
int bpd_build_tok_next(const int32_t* trans, int32_t num_states, int32_t num_symbols,
                       int32_t dead, const uint8_t* accept, const uint8_t* live,
                       const int32_t* tok_offsets, const uint8_t* tok_symbols,
                       int64_t vocab, int32_t eos_id, const int32_t* row_states,
                       int32_t num_rows, int32_t* out, void* stream);

/* bpd_build_reachability: live[s] = 1 iff an accepting state is reachable
 * from s through trans ([num_states * num_symbols], targets outside
 * [0, num_states) ignored); device pointers, at most 65536 states.  The
 * reference's build_reachability (fsa.py:70-104, the torch op of
 * torch_ops.cpp:95-107) and its sweep kernel (mask_cuda.cu:84-103, which its
 * op never reaches); bpd_host_build_reachability is the host form. */
int bpd_build_reachability(const int32_t* trans, int32_t num_states, int32_t num_symbols,
                           const uint8_t* accept, uint8_t* live, void* stream);
int bpd_host_build_reachability(const int32_t* trans, int32_t num_states, int32_t num_symbols,
                                const uint8_t* accept, uint8_t* live);

/* Symbol-class FSA walked per token on the device, without a tok_next table
 * (grammars too large to densify).  The reference's FsaTable + TokenSymbols
 * (mask.hpp:18-38) with the symbol classes narrowed to uint8.  The verdict
 * of (state s, token t) is step() of mask_cpu.cpp:53-71: EOS allowed iff
 * s >= 0 and accept[s]; otherwise s >= 0, every symbol < num_symbols, the
 * walk never meets `dead` (nor leaves [0, num_states)) and ends live. */
typedef struct BpdFsaTable {
  const int32_t* trans;       /* [num_states * num_symbols] */
  int32_t num_states, num_symbols, dead;
  const uint8_t* accept;      /* [num_states] */
  const uint8_t* live;        /* [num_states] */
  const int32_t* tok_offsets; /* [vocab + 1] */
  const uint8_t* tok_symbols; /* [tok_offsets[vocab]] */
  int64_t vocab;
  int32_t eos_id;             /* -1: none */
  /* optional (NULL = none), read by bpd_fsa_advance: `trans` as uint16 with
   * every entry outside [0, num_states) or naming a state that is not live
   * set to 0xFFFF (a walk that reaches a non-live state can only end
   * rejected); needs num_states < 65535 */
  const uint16_t* trans16;    /* [num_states * num_symbols] */
  /* optional (NULL = none), read by bpd_fsa_advance: per token 16 bytes,
   * its first 15 symbol classes (zero padded) and min(length, 255) */
  const uint8_t* tok_records; /* [vocab * 16] */
} BpdFsaTable;

/* bpd_fsa_apply_mask: logits[b, t] = neg_inf (checked conversion as in
 * bpd_dense_apply_mask) iff token t is rejected from state(b) =
 * states[slots ? slots[b] : b]; every entry of a row with state(b) < 0 is
 * rejected, and so is every entry of a row whose state is >= num_states
 * (BPD_FLAG_STATE_RANGE set in err).  Any float dtype.  Replaces
 * apply_mask_batch_cuda (mask.hpp:107-113) behind torch_ops.cpp:109-152. */
int bpd_fsa_apply_mask(const BpdFsaTable* table, void* logits, int dtype, int64_t rows, int64_t ld,
                       const int32_t* states, const int64_t* slots, double neg_inf, int32_t* err,
                       void* stream);

/* bpd_fsa_compute_mask: packed allow bits [rows, ceil(vocab/32)], LSB-first.
 * Replaces compute_mask_batch_cuda (mask.hpp:91-97, torch_ops.cpp:154-189). */
int bpd_fsa_compute_mask(const BpdFsaTable* table, const int32_t* states, const int64_t* slots,
                         int64_t rows, uint32_t* bits, int32_t* err, void* stream);

/* bpd_fsa_advance: next_out[b] = step(state(b), t(b)) (-1 off a valid path),
 * t(b) read as in bpd_dense_advance (int32 or int64, negative ids indexing
 * from the end); with write_back the pool slot is updated too.  `pending`
 * (num_pending <= BPD_MAX_FUSED_PENDING queued pool writes: slots, then
 * values) is applied as in bpd_dense_advance: a row whose slot has a queued
 * write starts from that value, and the writes land before the rows write
 * back.  Up to 4096 rows run as one fused launch (the table staged in LDS
 * when it fits); larger batches take no queued writes and need next_out.
 * Replaces advance_state_batch_cuda (mask.hpp:99-105, torch_ops.cpp:191-229)
 * and, with the queued writes, ConstraintBatch.commit's pool update
 * (batch.py:206-215) for bundles without tok_next. */
int bpd_fsa_advance(const BpdFsaTable* table, int32_t* states, const int64_t* slots,
                    const int64_t* pending, int64_t num_pending, const void* tokens,
                    int token_dtype, int64_t rows, int32_t* next_out, int write_back,
                    int32_t* err, void* stream);

/* Host (CPU-tensor) forms of the dense entry points. */
int bpd_host_dense_apply_mask(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                              const int32_t* tok_next, int32_t num_states,
                              const int32_t* states, const int64_t* slots, double neg_inf);
/* bpd_host_dense_apply_mask_bits: the host twin of bpd_dense_apply_mask_bits
 * (the mask from the packed allow-bit table; no queued writes): the CPU
 * branch of apply_mask_ (ops.py:271-276), reading V/8 bytes of table per row
 * instead of 4V. */
int bpd_host_dense_apply_mask_bits(void* logits, int dtype, int64_t rows, int64_t vocab,
                                   int64_t ld, const uint32_t* allow_bits, int64_t words,
                                   int32_t num_states, const int32_t* states,
                                   const int64_t* slots, double neg_inf);
int bpd_host_dense_advance(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                           int32_t* states, const int64_t* slots, const void* tokens,
                           int token_dtype, int64_t rows, int32_t* next_out, int write_back);
int bpd_host_dense_compute_mask(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                const int32_t* states, const int64_t* slots, int64_t rows,
                                uint32_t* bits);
int bpd_host_build_tok_next(const int32_t* trans, int32_t num_states, int32_t num_symbols,
                            int32_t dead, const uint8_t* accept, const uint8_t* live,
                            const int32_t* tok_offsets, const uint8_t* tok_symbols,
                            int64_t vocab, int32_t eos_id, const int32_t* row_states,
                            int32_t num_rows, int32_t* out);

/* bpd_stage_int64: enqueue a copy of n int64 values from host memory `src`
 * (any memory; free to change once the call returns) to device memory `dst`
 * on `stream`, through a per-stream ring of pinned buffers (a buffer is
 * reused once the copy that last read it has completed).  The per-step
 * upload of slot lists and queued pool writes; no counterpart in the
 * reference, whose batch classes build a device tensor per call
 * (batch.py:176-190, 206-215). */
int bpd_stage_int64(int64_t* dst, const int64_t* src, int64_t n, void* stream);

/* ------------------------------------------------------------------ PDA --
 * Flattened grammar (grammar/device.py:79-158, pda.hpp:46-69): every rule's
 * NFA in one global state space plus a CSR edge list.  The same struct
 * carries host pointers for bpd_host_* / bpd_pda_init and device pointers for
 * the device entry points.
 */
typedef struct BpdPdaTable {
  int32_t num_states;
  int32_t root_start;
  int32_t root_accept;
  int32_t num_edges;
  const uint8_t* accept;       /* [num_states] */
  const uint8_t* live;         /* [num_states] */
  const int32_t* edge_offsets; /* [num_states + 1] */
  const int32_t* edge_kind;    /* [num_edges] BPD_PDA_EDGE_* */
  const int32_t* edge_lo;      /* [num_edges] */
  const int32_t* edge_hi;      /* [num_edges] */
  const int32_t* edge_dst;     /* [num_edges] */
  const int32_t* edge_callee;  /* [num_edges] */
} BpdPdaTable;

/* Frame lists of the device mask's fast path (no counterpart in the
 * reference: an acceleration of pda_try_token, pda.hpp:248-258).  A list is
 * an ordered list of n <= 8 config suffixes, each of 1..BPD_PDA_FRAME_SUFFIX
 * frames: keys[l] = {n, the n suffix lengths (0 past n), then suffix i's
 * frames at words 9 + BPD_PDA_FRAME_SUFFIX * i .., 0 elsewhere}.  A config-set
 * whose configs are a common stack P followed by list l's suffixes (in
 * config order, every depth within BPD_PDA_MAX_DEPTH after
 * BPD_PDA_FRAME_SUFFIX more frames on P) steps exactly like the list while no
 * config pops into P and no suffix grows past BPD_PDA_FRAME_SUFFIX frames.
 * Such a row takes its verdicts from allowed[l] (bit t of word t / 32: every
 * byte of token t leads to a list) and walks only the tokens at walk
 * positions seeds[seed_off[l] .. seed_off[l + 1]) (the tokens that meet a
 * boundary, EOS and the empty tokens; every other token not in allowed[l]
 * is rejected).  trans[l][c] is the list byte c leads to (or-ed with
 * BPD_PDA_FRAME_SAT when the step drops a config at the 8-config cap, and
 * with BPD_PDA_FRAME_RAW when its compaction drops none: a set stepped by
 * the byte then holds exactly the words composed from the list's key, every
 * word past the configs' frames 0), -1
 * when it empties the set, -2 at a boundary: the device fills the
 * transition-table row of every such set it meets (a byte that keeps the
 * list and the saturation flag leads back to the set, a byte that empties
 * it is dead) without stepping it.  slots is an open-addressing table of the
 * keys: the probe for a list starts at slot h & (BPD_PDA_FRAME_SLOTS - 1) of
 * its hash h (grammar/frames.py list_hash) and ends at the first
 * BPD_PDA_FRAME_EMPTY slot; a slot holds l | ((h >> 10) & 0xFFFFF) << 12.
 * The device matches a set at its longest common stack below every top and
 * up to BPD_PDA_FRAME_SUFFIX - 1 frames less.  Built by grammar/frames.py
 * for the default walk order: the device trusts the contents (seed_off
 * non-decreasing within the seeds array; wrong lists give wrong verdicts). */
#define BPD_PDA_MAX_FRAME_LISTS 1400
#define BPD_PDA_FRAME_SLOTS 2048
#define BPD_PDA_FRAME_SUFFIX 5
#define BPD_PDA_FRAME_KEY_WORDS 56
#define BPD_PDA_FRAME_SAT 0x10000
#define BPD_PDA_FRAME_RAW 0x20000
#define BPD_PDA_FRAME_EMPTY 0xFFFFFFFFu
typedef struct BpdPdaFrames {
  int32_t num_lists;       /* 0 .. BPD_PDA_MAX_FRAME_LISTS */
  int32_t words;           /* (vocab_size + 31) / 32 */
  const int32_t* keys;     /* [num_lists, BPD_PDA_FRAME_KEY_WORDS] */
  const uint32_t* slots;   /* [BPD_PDA_FRAME_SLOTS] */
  const int32_t* trans;    /* [num_lists, 256] */
  const uint32_t* allowed; /* [num_lists, words] */
  const int32_t* seed_off; /* [num_lists + 1] */
  const int32_t* seeds;    /* [seed_off[num_lists]] walk positions */
} BpdPdaFrames;

typedef struct BpdTokenBytes {
  int32_t vocab_size;
  int32_t eos_id;
  const int32_t* offsets; /* [vocab_size + 1] */
  const uint8_t* bytes;   /* [offsets[vocab_size]] */
  /* optional (NULL = id order): a permutation of the token ids; the
   * memoised device mask walks tokens in this order, consecutive lanes of a
   * wave at consecutive positions (any permutation gives the same verdicts;
   * by first byte, length, then bytes, lanes walk similar tokens) */
  const int32_t* order;
  /* optional (NULL = none; ignored without `order`): [257] first-byte runs
   * of `order`: walk positions [runs[c], runs[c + 1]) hold exactly the
   * tokens of first byte c (c < 256; the run of c = 255 ends at runs[256]),
   * [runs[256], vocab_size) the EOS token and the empty tokens.  The device
   * mask skips the run of every byte that empties a row's config-set. */
  const int32_t* runs;
  /* optional (NULL = none): frame lists for `order` (device pointers inside
   * a host struct) */
  const BpdPdaFrames* frames;
  /* optional (0 = none): a tag that identifies the contents of offsets,
   * bytes and order.  The device mask packs the token records into its
   * workspace unless the workspace header already carries this tag for the
   * same row count (a workspace keeps them between calls): by a launch of
   * its own the first time the process masks with the tag on the
   * workspace, inside the mask after that.  Zero the first 256 bytes of a
   * newly allocated workspace: the header also holds the mask's finish
   * count and deferred-write slots, and a slot is trusted when it carries
   * the launch's generation (never 0). */
  uint64_t pack_tag;
} BpdTokenBytes;

/* bpd_pda_init: the closed initial config-set (pda.hpp:200-207), host only,
 * as the reference's pda_init op (torch_ops.cpp:307-324). */
int bpd_pda_init(const BpdPdaTable* g, int32_t* config_out);

/* bpd_pda_feed: host only; consume `n` raw bytes into one config-set in place
 * (pda_advance_byte per byte, pda.hpp:211-236).  Returns 1 when every byte
 * kept the set non-empty (config updated), 0 when a byte emptied it (config
 * untouched), or a negative error code.  Seeds a row with a known prefix; no
 * single reference entry point corresponds (the reference's tests feed bytes
 * through pda_advance_byte directly, test_pda.cpp:46-51). */
int bpd_pda_feed(const BpdPdaTable* g, int32_t* config, const uint8_t* data, int64_t n);

/* bpd_host_frame_lists: host only (no counterpart in the reference: it
 * builds the frame lists of BpdPdaFrames).  Enumerates the stack-relative
 * config lists of the tables breadth first from the closure of every single
 * state (at most max_lists <= BPD_PDA_MAX_FRAME_LISTS) and writes their keys
 * [max_lists, BPD_PDA_FRAME_KEY_WORDS], byte transitions [max_lists, 256]
 * and the keys' slot table [BPD_PDA_FRAME_SLOTS]; returns the number of
 * lists, or a negative error code. */
int bpd_host_frame_lists(const BpdPdaTable* g, int32_t max_lists, int32_t* keys, int32_t* trans,
                         uint32_t* slots);

/* bpd_frame_classify: bpd_host_frame_classify on the device, in two passes
 * on `stream` (device pointers).  Count pass (block_offsets NULL): `allowed`
 * (zeroed by the caller) gets the inside tokens and block_counts
 * [num_lists, bpd_frame_classify_blocks(vocab_size)] the seeds of each
 * list's block of walk positions.  Fill pass: with block_offsets the
 * exclusive prefix sums of those counts in the same order (int64), seeds
 * gets each list's seeds in walk order at its offsets. */
int bpd_frame_classify(const int32_t* trans, int32_t num_lists, const int32_t* tok_offsets,
                       const uint8_t* tok_bytes, int32_t vocab_size, int32_t eos_id, const int32_t* order,
                       uint32_t* allowed, int32_t* block_counts, const int64_t* block_offsets,
                       int32_t* seeds, void* stream);
int32_t bpd_frame_classify_blocks(int32_t vocab_size);

/* bpd_host_frame_classify: host only (no counterpart in the reference: it
 * builds the frame lists' bitmaps and seeds, BpdPdaFrames).  Walks every
 * token from every list through trans [num_lists, 256] on up to `threads`
 * host threads: allowed [num_lists, (vocab_size + 31) / 32] gets the inside
 * tokens, seed_count [num_lists] the number of seeds of each list, and, when
 * seed_off [num_lists + 1] (offsets matching those counts) and seeds are
 * given, seeds the walk positions in `order` of each list's seeds,
 * ascending. */
int bpd_host_frame_classify(const int32_t* trans, int32_t num_lists, const int32_t* tok_offsets,
                            const uint8_t* tok_bytes, int32_t vocab_size, int32_t eos_id,
                            const int32_t* order, uint32_t* allowed, int32_t* seed_count,
                            const int32_t* seed_off, int32_t* seeds, int32_t threads);

/* bpd_pda_apply_mask: logits[b, t] = neg_inf unless token t is accepted from
 * config-set configs[row(b)] (pda_try_token, pda.hpp:248-258), or for every t
 * when broken[row(b)] != 0 (broken may be NULL).  row(b) = slots ? slots[b]
 * : b.  Replaces pda_apply_mask_op (torch_ops.cpp:326-376) and the broken-row
 * fill of CFGConstraintBatch.apply_mask (device.py:252-266). */
size_t bpd_pda_workspace_bytes(int64_t rows, int32_t vocab);
int bpd_pda_apply_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                       const int32_t* configs, const int64_t* slots, const uint8_t* broken,
                       int64_t rows, void* logits, int dtype, int64_t ld, double neg_inf,
                       void* workspace, size_t workspace_bytes, void* stream);

/* bpd_pda_compute_mask: packed allow bits (compute_mask_pda_batch,
 * pda_cpu.cpp:7-21). */
int bpd_pda_compute_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                         const int32_t* configs, const int64_t* slots, int64_t rows,
                         uint32_t* bits, void* workspace, size_t workspace_bytes,
                         void* stream);

/* bpd_pda_advance: advance configs[row(b)] in place by tokens[b]; ok[b] = 0 and
 * the config-set untouched when the token is rejected; EOS only tests
 * completeness (advance_state_pda_batch, pda_cpu.cpp:35-54).  With broken
 * non-NULL, broken[row(b)] |= !ok[b] and status[b] = broken[row(b)] ? -1 : 1
 * (CFGConstraintBatch.commit, device.py:268-283); without it status[b] =
 * ok[b] ? 1 : -1.  ok, broken and status may each be NULL.  With the
 * workspace of the preceding bpd_pda_apply_mask / bpd_pda_compute_mask of the
 * same rows (bpd_pda_workspace_bytes(rows, vocab) bytes, same stream), the
 * token is walked through the transition tables that call built, and only
 * its last byte is stepped; results are identical (raw words included). */
int bpd_pda_advance(const BpdPdaTable* g, const BpdTokenBytes* toks, int32_t* configs,
                    const int64_t* slots, const void* tokens, int token_dtype, int64_t rows,
                    uint8_t* ok, uint8_t* broken, int32_t* status, int32_t* err,
                    void* workspace, size_t workspace_bytes, void* stream);

int bpd_host_pda_apply_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                            const int32_t* configs, const int64_t* slots,
                            const uint8_t* broken, int64_t rows, void* logits, int dtype,
                            int64_t ld, double neg_inf);
int bpd_host_pda_compute_mask(const BpdPdaTable* g, const BpdTokenBytes* toks,
                              const int32_t* configs, const int64_t* slots, int64_t rows,
                              uint32_t* bits);
int bpd_host_pda_advance(const BpdPdaTable* g, const BpdTokenBytes* toks, int32_t* configs,
                         const int64_t* slots, const void* tokens, int token_dtype,
                         int64_t rows, uint8_t* ok, uint8_t* broken, int32_t* status);

/* ----------------------------------------------------------------- soft --
 * bpd_soft_build_lookahead: the uniform-count bias table of build_lookahead
 * (ops.py:200-236), float32 [num_states, vocab]: k-1 rounds of
 * logZ(s) = logsumexp_t logZ(tok_next[s, t]) (logaddexp with 0 for accepting
 * s, -inf off the live set), then out[s, t] = logZ(tok_next[s, t]), -inf on
 * rejected tokens, 0 / -inf in the EOS column.  Workspace:
 * bpd_soft_workspace_bytes(0, num_states, k).
 */
size_t bpd_soft_workspace_bytes(int64_t rows, int32_t num_states, int32_t k);
int bpd_soft_build_lookahead(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                             const uint8_t* accept, const uint8_t* live, int32_t eos_id, int32_t k,
                             float* out, void* workspace, size_t workspace_bytes, void* stream);

/* bpd_soft_apply: logits[b, t] += alpha * lookahead[state(b), t] on finite
 * entries (float arithmetic, stored in the logits dtype) and -inf where the
 * lookahead is -inf or state(b) < 0 (apply_soft_, ops.py:239-259, called by
 * ConstraintBatch.apply_soft, batch.py:192-204). */
int bpd_soft_apply(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                   const float* lookahead, int32_t num_states, const int32_t* states,
                   const int64_t* slots, float alpha, int32_t* err, void* stream);

int bpd_host_soft_build_lookahead(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                                  const uint8_t* accept, const uint8_t* live, int32_t eos_id,
                                  int32_t k, float* out);
int bpd_host_soft_apply(void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                        const float* lookahead, int32_t num_states, const int32_t* states,
                        const int64_t* slots, float alpha);

/* --------------------------------------------------- prior-weighted soft --
 * The reference's build_lookahead (ops.py:200-236) counts continuations
 * uniformly; this variant weights them by each row's own model prior
 * logpi_b = log_softmax(logits_b) and replaces the float32 logits in place:
 *   logZ_0(s) = 0 on live s; k-1 rounds of
 *   logZ(s) = logsumexp_t [logpi_b(t) + logZ(tok_next[s, t])]
 *             (logaddexp with logpi_b(eos) for accepting s), -inf off live;
 *   out[b, t] = logpi_b(t) + alpha * logZ(tok_next[s_b, t]) on allowed t,
 *   logpi_b(eos) / -inf in the EOS column for accepting / other s_b, -inf on
 *   every other entry and on rows with s_b < 0.
 * With logpi == 0 the rounds are the reference's uniform ones.  The reference
 * has no such kernel: its model-weighted scoring (lookahead.py:57-70,
 * logit + alpha * log P(valid continuation)) takes a forward pass per
 * candidate instead of the current row's prior.
 *
 * bpd_host_soft_classes groups tokens with equal tok_next columns (once per
 * grammar, host memory): class c is class_tok[class_off[c] .. class_off[c+1]),
 * cut into pieces piece_off[p] .. piece_off[p+1] of at most 256 members, its
 * pieces being class_piece[c] .. class_piece[c+1]; the (class, next state)
 * pairs of state s are pair_class / pair_next[state_off[s] .. state_off[s+1]);
 * token_class[t] is t's class, -1 for tokens rejected in every state;
 * token_class16, when given and num_classes < 65535, receives the same map
 * narrowed to uint16 (0xFFFF for -1).  Called with any of the int32 arrays
 * null it only sets the counts; called again with arrays of those sizes
 * (counts left in place) it fills them.
 *
 * bpd_soft_prior takes the same struct with the arrays copied to the device;
 * with token_class16 set its statistics pass reads the narrow map instead of
 * token_class.
 * Workspace: bpd_soft_prior_workspace_bytes(rows, vocab, num_classes, num_pieces)
 * bytes (no initial contents needed; calls that overlap on one workspace race).
 */
typedef struct BpdSoftClasses {
  int32_t num_classes, num_members, num_pieces, num_pairs;
  int32_t* class_off;   /* [num_classes + 1] */
  int32_t* class_tok;   /* [num_members] */
  int32_t* class_piece; /* [num_classes + 1] */
  int32_t* piece_off;   /* [num_pieces + 1] */
  int32_t* state_off;   /* [num_states + 1] */
  int32_t* pair_class;  /* [num_pairs] */
  int32_t* pair_next;   /* [num_pairs] */
  int32_t* token_class; /* [vocab] */
  uint16_t* token_class16; /* [vocab] optional: token_class as uint16, 0xFFFF for -1 */
  /* optional: the classed tokens of each BPD_SOFT_MEMBER_CHUNK-token chunk of
   * the vocab, in token order, as (offset in chunk << 16 | class), padded
   * with 0xFFFFFFFF to chunk_cap entries per chunk.  The caller provides
   * ceil(vocab / BPD_SOFT_MEMBER_CHUNK) * BPD_SOFT_MEMBER_CAP_MAX entries; the
   * builder sets chunk_cap (256, 512 or 1024), or 0 when a chunk holds more
   * classed tokens than that or there are 65535 classes or more (the list is
   * then unused). */
  uint32_t* chunk_members;
  int32_t chunk_cap;
} BpdSoftClasses;

#define BPD_SOFT_MEMBER_CHUNK 4096
#define BPD_SOFT_MEMBER_CAP_MAX 1024

int bpd_host_soft_classes(const int32_t* tok_next, int32_t num_states, int64_t vocab,
                          BpdSoftClasses* out);
size_t bpd_soft_prior_workspace_bytes(int64_t rows, int64_t vocab, int32_t num_classes,
                                      int32_t num_pieces);
int bpd_soft_prior(float* logits, int64_t rows, int64_t vocab, int64_t ld, int32_t num_states,
                   const uint8_t* accept, const uint8_t* live, int32_t eos_id,
                   const int32_t* states, const int64_t* slots, const BpdSoftClasses* classes,
                   int32_t k, float alpha, void* workspace, size_t workspace_bytes, int32_t* err,
                   void* stream);
int bpd_host_soft_prior(float* logits, int64_t rows, int64_t vocab, int64_t ld,
                        const int32_t* tok_next, int32_t num_states, const uint8_t* accept,
                        const uint8_t* live, int32_t eos_id, const int32_t* states,
                        const int64_t* slots, int32_t k, float alpha);

/* bpd_soft_prior_noalloc: bpd_soft_prior without a workspace argument and
 * without any allocation: its workspace is a file-scope device array of
 * BPD_SOFT_PRIOR_SCRATCH_BYTES per GPU (held until the process ends; its
 * address is looked up once per device on the first call there).  No
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory -- code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc.  Calls needing more workspace than the array holds
 * (bpd_soft_prior_workspace_bytes > BPD_SOFT_PRIOR_SCRATCH_BYTES, e.g. more
 * than 428 rows at the email DFA's 126 classes over a 151,936-token
 * vocabulary) fail with BPD_ERR_INVALID.
 * Results equal bpd_soft_prior's.  Every call on one GPU uses the same array:
 * calls that overlap on one GPU (several streams or threads) race and must
 * be serialised by the caller.  Nothing in the array has to start at zero
 * (each launch writes every word it reads), so it is never cleared. */
#define BPD_SOFT_PRIOR_SCRATCH_BYTES (16 << 20)
int bpd_soft_prior_noalloc(float* logits, int64_t rows, int64_t vocab, int64_t ld,
                           int32_t num_states, const uint8_t* accept, const uint8_t* live,
                           int32_t eos_id, const int32_t* states, const int64_t* slots,
                           const BpdSoftClasses* classes, int32_t k, float alpha, int32_t* err,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BPDECODE_HIP_H_ */
