/*
 * grammar_oracle.h — CPU restatement of the reference's grammar-mask production.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker of strim_grammar_*). Only tests/ load it.
 * Semantics and reference lines: grammar_oracle.c.
 */
#ifndef STRIM_GRAMMAR_ORACLE_H
#define STRIM_GRAMMAR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct so_trie so_trie;

/* the vocabulary trie (GrammarVocab.init): tokens with empty bytes or skip[i] != 0 left out */
so_trie* so_trie_build(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                       const uint8_t* skip);
void so_trie_free(so_trie* t);
int32_t so_trie_nodes(const so_trie* t);

/* mask words of a key (GrammarRuntime.mask; free / forced keys as DeviceMasks.all / only) */
void so_grammar_mask(const so_trie* t, int32_t width, const int32_t* eos, int32_t n_eos,
                     int32_t n_states, const int32_t* next, const uint8_t* flags, int32_t key,
                     uint32_t* out_words);

/* GrammarRuntime.advance: -1 (dead) as soon as a byte has no transition */
int32_t so_grammar_advance_bytes(int32_t s, const uint8_t* b, uint32_t len,
                                 const int32_t* next);

/* keys of the k + 1 verify rows per request (RequestConstraint.verifyMask's walk) */
void so_grammar_verify_keys(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                            int32_t n_states, const int32_t* next, const int32_t* state,
                            int32_t B, const int32_t* tokens, int32_t k, int32_t* keys_out);

/* RequestConstraint.State with its constants: {g, in_think, count, budget, close_id,
 * violated}, six int32 per request (the layout of strim_request_state) */
typedef struct {
  int32_t g, in_think, count, budget, close_id, violated;
} so_request_state;

/* RequestConstraint.key / verifyMask (RequestConstraint.swift:85-92,134-145): the key of
 * each request's next row and of its k verify rows */
void so_request_keys(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                     int32_t n_states, const int32_t* next, const so_request_state* states,
                     int32_t B, const int32_t* drafts, int32_t k, int32_t* keys_out);

/* RequestConstraint.advance (RequestConstraint.swift:104-109) over drafts[0 .. accepted)
 * and then last, per request (accepted NULL: none; last < 0: no step) */
void so_request_advance(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                        int32_t n_states, const int32_t* next, so_request_state* states,
                        int32_t B, const int32_t* drafts, int32_t k, const int32_t* accepted,
                        const int32_t* last);

#ifdef __cplusplus
}
#endif

#endif /* STRIM_GRAMMAR_ORACLE_H */
