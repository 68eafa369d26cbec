/*
 * strim_grammar.h — on-device grammar-mask production for the token-selection path.
 *
 * The reference builds a token mask on the host: a byte trie over the tokenizer vocabulary
 * is walked through the grammar's DFA for each state, cached as a bitset per state and
 * expanded into a bool array per upload (GrammarVocab.swift:3-113,
 * RequestConstraint.swift:5-60). Here the vocabulary bytes, the DFA transition table and
 * the per-state mask cache live in HBM. A mask row is produced by one launch straight into
 * the packed u32 words that strim_sample / strim_verify read (bit i of word w allows token
 * 32 w + i), and the verify rows' states are stepped by the drafts' bytes on the device.
 *
 * Row keys (RequestConstraint.Key, RequestConstraint.swift:65,85-92,113-119):
 *   key >= 0    grammar state `key`: the tokens whose bytes keep the DFA alive from it,
 *               when the state consumes, plus the end-of-turn ids when it accepts;
 *   key == -1   free: every token below width allowed;
 *   key <= -2   forced: only token (-2 - key) allowed (the thinking-budget close id).
 * A state at or above the table's state count gives an all-zero row, which strim_sample
 * reports as STRIM_EEMPTY.
 *
 * One table holds every program's states (state ids are global), so a batch whose
 * requests follow different grammars takes its masks from one call. The table grows:
 * strim_grammar_append_states adds states without touching the cached masks, and a
 * transition may be left unknown (STRIM_DFA_UNKNOWN) until the host has interned its
 * target, as the reference's lazily built DFA does (GrammarDFA.swift:36-58). A walk that
 * meets an unknown transition records the (state, byte) pair; strim_grammar_pending hands
 * the pairs to the host, which interns the targets and fills the entries with
 * strim_grammar_set_next. A mask row whose walk met one is incomplete (it is not cached,
 * and its bits for the tokens that met one are 0) and must be produced again after the
 * pairs are filled; a key walk that meets one gives STRIM_GRAMMAR_UNRESOLVED, a key whose
 * row is all zero.
 *
 * All calls are stream-ordered; keys, tokens and outputs are device memory. Calls on one
 * strim_grammar must not overlap (issue them on one stream): a mask call reads the cached
 * blocks earlier calls produced, and one running alongside could read a block that is
 * still being written.
 */
#ifndef STRIM_GRAMMAR_H
#define STRIM_GRAMMAR_H

#include <stdint.h>

#include "strim_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct strim_grammar strim_grammar;

#define STRIM_DFA_ACCEPTING 1 /* flags bit: the state may end (GrammarDFA.accepting)     */
#define STRIM_DFA_CONSUMING 2 /* flags bit: the state can take bytes (GrammarDFA.consuming) */
#define STRIM_DFA_DEAD (-1)    /* table entry: the byte kills every stack                  */
#define STRIM_DFA_UNKNOWN (-2) /* table entry: not interned yet (GrammarDFA.unknown)       */
#define STRIM_GRAMMAR_UNRESOLVED 0x7FFFFFFF /* key after an unknown transition (zero row) */

/* Uploads the vocabulary (replaces GrammarVocab.init, GrammarVocab.swift:16-51, and the
 * GrammarEngine construction, GrammarVocab.swift:116-130).
 *   count       tokens with byte strings; token i has bytes[offsets[i] .. offsets[i+1])
 *               (host arrays, offsets non-decreasing, offsets[0] = 0)
 *   skip        host [count] or NULL: nonzero ids never appear in a grammar mask
 *               (control tokens); empty byte strings never appear either
 *   width       logits width, the mask's bit count (ids at or above width are dropped)
 *   eos, n_eos  host end-of-turn ids, allowed in an accepting state's mask
 *   cache_slots mask rows kept in HBM (width / 8 bytes each: the cache's byte budget,
 *               as the reference bounds its masks, GrammarVocab.swift:124,150-156, and
 *               DeviceMasks.capacity, RequestConstraint.swift:12,35-43). Any state may
 *               occupy a slot, block by block: state s maps to the two slots of set
 *               s mod (cache_slots / 2) and replaces the one stored first (DeviceMasks'
 *               insertion order), except a slot holding a state that the same call
 *               reads. 0 or 1: no cache
 * The table is empty until strim_grammar_set_dfa or strim_grammar_append_states. */
int strim_grammar_create(strim_grammar** out, int32_t device, int32_t count,
                         const uint32_t* offsets, const uint8_t* bytes, const uint8_t* skip,
                         int32_t width, const int32_t* eos, int32_t n_eos,
                         int32_t cache_slots);
int strim_grammar_destroy(strim_grammar* g);

/* Replaces the whole table with one DFA (the compiled GrammarDFA of GrammarRuntime.init,
 * GrammarVocab.swift:57-69, GrammarDFA.swift:13-58) and clears the mask cache and the
 * pending pairs.
 *   next   host [n_states][256]: the state after byte b, STRIM_DFA_DEAD, or
 *          STRIM_DFA_UNKNOWN
 *   flags  host [n_states]: STRIM_DFA_ACCEPTING | STRIM_DFA_CONSUMING
 * Returns STRIM_EINVAL for an entry outside [-2, n_states) or more than 2^23 states. */
int strim_grammar_set_dfa(strim_grammar* g, void* stream, int32_t n_states,
                          const int32_t* next, const uint8_t* flags);

/* Appends n_new states to the table (GrammarDFA.intern, GrammarDFA.swift:47-58, for one
 * or several programs): they take ids first .. first + n_new - 1, with *first_out =
 * first = the previous state count. Cached masks stay valid (a known entry never
 * changes). next host [n_new][256] with entries in [-2, first + n_new) (global ids),
 * flags host [n_new]. Returns STRIM_EINVAL for a bad entry, STRIM_ECAPACITY past 2^23
 * states. Synchronises the stream. */
int strim_grammar_append_states(strim_grammar* g, void* stream, int32_t n_new,
                                const int32_t* next, const uint8_t* flags, int32_t* first_out);

/* Fills unknown entries (GrammarDFA.next memoising a transition, GrammarDFA.swift:36-45):
 * entry where[i] = state * 256 + byte becomes to[i] (a state id or STRIM_DFA_DEAD). Only
 * an unknown entry may change; setting a known entry to another value fails with
 * STRIM_EINVAL (cached masks depend on it) and sets nothing. where, to host [n].
 * Synchronises the stream. */
int strim_grammar_set_next(strim_grammar* g, void* stream, int32_t n, const int64_t* where,
                           const int32_t* to);

/* The unknown transitions that walks met since the last call: up to cap entries
 * state * 256 + byte into out (host), *n_out = how many were recorded (each pair once;
 * more than cap: call again after filling these). The pairs handed out are forgotten;
 * a walk that meets one again records it again. Synchronises the stream. */
int strim_grammar_pending(strim_grammar* g, void* stream, int64_t* out, int32_t cap,
                          int32_t* n_out);

/* Forgets the cached mask rows of states [first, first + n) (GrammarEngine.trim dropping
 * a program's masks, GrammarVocab.swift:150-156); their slots are reused first. */
int strim_grammar_drop_masks(strim_grammar* g, void* stream, int32_t first, int32_t n);

/* Mask rows for n keys (replaces GrammarRuntime.mask, GrammarVocab.swift:75-102, and
 * DeviceMasks.allowed / only / all with their bool expansion,
 * RequestConstraint.swift:16-58): out[r][0 .. ceil(width / 32)) packed words, out_stride
 * words apart. keys device [n]. Rows with equal keys are produced once and copied. */
int strim_grammar_masks(strim_grammar* g, void* stream, const int32_t* keys, int32_t n,
                        uint32_t* out, int64_t out_stride);

/* Verify-row keys (replaces RequestConstraint.verifyMask's key walk and
 * GrammarRuntime.advance, RequestConstraint.swift:94-102,134-145,
 * GrammarVocab.swift:107-112). For request b, keys_out[b][0] = key(state[b]) and
 * keys_out[b][i + 1] is the key after tokens[b][0 .. i]: each token's bytes step the
 * state; a step to dead makes that row and every later row free (-1). Free and forced
 * keys are left as they are: a key carries no thinking-phase state, so a request in its
 * thinking phase is walked with strim_request_keys below. Ids outside [0, count) have no
 * bytes and leave the state unchanged. state device [B] (keys), tokens device [B][k],
 * keys_out device [B][k + 1]. */
int strim_grammar_advance(strim_grammar* g, void* stream, const int32_t* state, int32_t B,
                          const int32_t* tokens, int32_t k, int32_t* keys_out);

/* ---- per-request constraint state ---------------------------------------------------
 * RequestConstraint.State and its constants (RequestConstraint.swift:62-83), one per
 * request in device memory. The key of a state (RequestConstraint.key, :85-92):
 *   in_think and budget >= 0 and count >= budget  -> forced(close_id)   (-2 - close_id)
 *   in_think otherwise                            -> free              (-1)
 *   g >= 0                                        -> grammar state g
 *   g < 0 (no grammar, or a step left it)         -> free
 * A step by token t (RequestConstraint.step, :94-102): in the thinking phase, t ==
 * close_id leaves it and any other token counts toward the budget; after it, a live
 * grammar state is stepped by t's bytes (dead = -1, so the request degrades to free). */
typedef struct strim_request_state {
  int32_t g;        /* grammar state, < 0 for none / dead                 (State.g)        */
  int32_t in_think; /* nonzero while the request is in its thinking phase (State.inThink)  */
  int32_t count;    /* thinking tokens emitted so far                     (State.count)    */
  int32_t budget;   /* thinking budget, < 0 for none                      (budget)         */
  int32_t close_id; /* the token that ends the thinking phase             (closeId)        */
  int32_t violated; /* set once an emitted token stepped the grammar dead (violated)       */
} strim_request_state;

/* Row keys of B requests without changing their states (RequestConstraint.key / verifyMask,
 * RequestConstraint.swift:85-92,121-126,134-145): keys_out[b][0] = key(states[b]) (the
 * next token's row) and keys_out[b][i + 1] the key after drafts[b][0 .. i]; once a draft
 * steps the grammar dead, that row and every later row are free. k = 0 (drafts NULL)
 * gives the next-token keys alone. states device [B], drafts device [B][k], keys_out
 * device [B][k + 1]; the keys feed strim_grammar_masks. */
int strim_request_keys(strim_grammar* g, void* stream, const strim_request_state* states,
                       int32_t B, const int32_t* drafts, int32_t k, int32_t* keys_out);

/* Steps each request by the tokens the engine emitted (RequestConstraint.advance,
 * RequestConstraint.swift:104-109): drafts[b][0 .. accepted[b]) and then last[b], the
 * outputs of strim_verify (accepted NULL: none, as after strim_sample, where k = 0 and
 * drafts may be NULL). accepted[b] is clamped to [0, k]; last[b] < 0 (a row error) steps
 * nothing. A grammar step to dead sets violated; the request is free from then on. */
int strim_request_advance(strim_grammar* g, void* stream, strim_request_state* states,
                          int32_t B, const int32_t* drafts, int32_t k, const int32_t* accepted,
                          const int32_t* last);

#ifdef __cplusplus
}
#endif

#endif /* STRIM_GRAMMAR_H */
