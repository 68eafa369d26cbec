/*
 * grammar_oracle.c — CPU restatement of the reference's grammar-mask production.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the library's grammar kernels. Only
 * tests/ may load it (through oracle.py); the product never does.
 *
 * It follows the reference's own algorithm, not the device one: a byte trie over the
 * vocabulary in preorder arrays (GrammarVocab.init, Sources/StrimEngine/GrammarVocab.swift:
 * 16-51) walked depth first through the DFA, marking every token whose trie node is reached
 * by live transitions and its byte-identical duplicates (GrammarRuntime.mask / walk,
 * GrammarVocab.swift:77-102); end-of-turn ids join the mask of an accepting state (:82).
 * advance feeds a token's bytes (GrammarVocab.swift:107-112) and the verify keys follow
 * RequestConstraint.verifyMask (Sources/StrimEngine/RequestConstraint.swift:134-145).
 *
 * Parity pins (tests/test_grammar.py): a brute-force per-token DFA walk in numpy on random
 * vocabularies and DFAs (an independent statement of the same set), the reference's
 * FakeVocab fixture (GrammarTests.swift:7-27) under hand-built DFAs with closed-form masks
 * (a one-literal grammar, a digits grammar, the empty-object prefix), and the
 * ConstraintRowTests.verifyRows rules (GrammarTests.swift:324-354) for the verify keys.
 *
 * Keys: >= 0 a DFA state, -1 free (all ids below width), <= -2 forced id (-2 - key);
 * a state at or above n_states gives an empty row.
 */
#include "grammar_oracle.h"

#include <stdlib.h>
#include <string.h>

struct so_trie {
  int32_t n_nodes;
  uint8_t* byte_of;      /* [n] byte on the edge into the node                       */
  int32_t* first_child;  /* [n]                                                      */
  int32_t* next_sib;     /* [n]                                                      */
  int32_t* token_at;     /* [n] first id whose bytes end here, -1 if none            */
  int32_t* dup_head;     /* [count] for a token_at id: first further id with its bytes */
  int32_t* dup_next;     /* [count] chain of byte-identical ids                      */
  int32_t count;
};

typedef struct {
  const uint8_t* p;
  uint32_t len;
  int32_t id;
} tok_ref;

/* lexicographic order of byte strings; a proper prefix sorts first; equal strings by id */
static int cmp_tok(const void* a, const void* b) {
  const tok_ref* x = (const tok_ref*)a;
  const tok_ref* y = (const tok_ref*)b;
  const uint32_t m = x->len < y->len ? x->len : y->len;
  const int c = m ? memcmp(x->p, y->p, m) : 0;
  if (c) return c;
  if (x->len != y->len) return x->len < y->len ? -1 : 1;
  return x->id < y->id ? -1 : (x->id > y->id);
}

so_trie* so_trie_build(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                       const uint8_t* skip) {
  tok_ref* order = (tok_ref*)malloc(sizeof(tok_ref) * (size_t)(count > 0 ? count : 1));
  int32_t n = 0;
  uint64_t total = 0;
  for (int32_t i = 0; i < count; ++i) {
    const uint32_t len = offsets[i + 1] - offsets[i];
    if (len == 0 || (skip && skip[i])) continue;
    order[n].p = bytes + offsets[i];
    order[n].len = len;
    order[n].id = i;
    ++n;
    total += len;
  }
  qsort(order, (size_t)n, sizeof(tok_ref), cmp_tok);
  so_trie* t = (so_trie*)calloc(1, sizeof(so_trie));
  const size_t cap = (size_t)total + 1;
  t->byte_of = (uint8_t*)malloc(cap);
  t->first_child = (int32_t*)malloc(cap * 4);
  t->next_sib = (int32_t*)malloc(cap * 4);
  t->token_at = (int32_t*)malloc(cap * 4);
  int32_t* last_child = (int32_t*)malloc(cap * 4);
  t->dup_head = (int32_t*)malloc(sizeof(int32_t) * (size_t)(count > 0 ? count : 1));
  t->dup_next = (int32_t*)malloc(sizeof(int32_t) * (size_t)(count > 0 ? count : 1));
  for (int32_t i = 0; i < count; ++i) t->dup_head[i] = t->dup_next[i] = -1;
  t->count = count;
  /* node 0 is the root */
  t->byte_of[0] = 0;
  t->first_child[0] = t->next_sib[0] = t->token_at[0] = last_child[0] = -1;
  int32_t nn = 1;
  uint32_t maxlen = 0;
  for (int32_t q = 0; q < n; ++q) maxlen = order[q].len > maxlen ? order[q].len : maxlen;
  int32_t* path = (int32_t*)malloc(sizeof(int32_t) * (maxlen + 1));
  int32_t depth = 0;  /* path[0 .. depth] is the previous token's node chain */
  path[0] = 0;
  const uint8_t* prev = NULL;
  uint32_t prev_len = 0;
  for (int32_t q = 0; q < n; ++q) {
    const tok_ref* tk = &order[q];
    uint32_t l = 0;
    const uint32_t m = prev_len < tk->len ? prev_len : tk->len;
    while (l < m && prev[l] == tk->p[l]) ++l;
    depth = (int32_t)l;  /* keep the shared prefix of the path */
    for (uint32_t d = l; d < tk->len; ++d) {
      const int32_t node = nn++;
      t->byte_of[node] = tk->p[d];
      t->first_child[node] = t->next_sib[node] = t->token_at[node] = last_child[node] = -1;
      const int32_t par = path[depth];
      if (t->first_child[par] < 0) t->first_child[par] = node;
      else t->next_sib[last_child[par]] = node;
      last_child[par] = node;
      path[++depth] = node;
    }
    const int32_t end = path[depth];
    if (t->token_at[end] < 0) {
      t->token_at[end] = tk->id;
    } else {
      /* append to the duplicate chain of the node's token */
      const int32_t head = t->token_at[end];
      if (t->dup_head[head] < 0) {
        t->dup_head[head] = tk->id;
      } else {
        int32_t c = t->dup_head[head];
        while (t->dup_next[c] >= 0) c = t->dup_next[c];
        t->dup_next[c] = tk->id;
      }
    }
    prev = tk->p;
    prev_len = tk->len;
  }
  t->n_nodes = nn;
  free(path);
  free(last_child);
  free(order);
  return t;
}

void so_trie_free(so_trie* t) {
  if (!t) return;
  free(t->byte_of);
  free(t->first_child);
  free(t->next_sib);
  free(t->token_at);
  free(t->dup_head);
  free(t->dup_next);
  free(t);
}

int32_t so_trie_nodes(const so_trie* t) { return t->n_nodes; }

static void set_bit(uint32_t* w, int32_t id, int32_t width) {
  if (id >= 0 && id < width) w[id >> 5] |= 1u << (id & 31);
}

/* depth-first walk from the root in state s (GrammarVocab.swift:88-102), iterative */
static void walk(const so_trie* t, int32_t s, const int32_t* next, int32_t width,
                 uint32_t* w) {
  typedef struct { int32_t child; int32_t state; } frame;
  frame* stack = (frame*)malloc(sizeof(frame) * (size_t)(t->n_nodes + 1));
  int32_t sp = 0;
  stack[sp].child = t->first_child[0];
  stack[sp].state = s;
  ++sp;
  while (sp > 0) {
    frame* f = &stack[sp - 1];
    const int32_t c = f->child;
    if (c < 0) { --sp; continue; }
    f->child = t->next_sib[c];  /* the sibling is visited after c's subtree */
    const int32_t nt = next[(int64_t)f->state * 256 + t->byte_of[c]];
    if (nt < 0) continue;
    const int32_t id = t->token_at[c];
    if (id >= 0 && id < width) {
      set_bit(w, id, width);
      for (int32_t d = t->dup_head[id]; d >= 0; d = t->dup_next[d]) set_bit(w, d, width);
    }
    if (t->first_child[c] >= 0) {
      stack[sp].child = t->first_child[c];
      stack[sp].state = nt;
      ++sp;
    }
  }
  free(stack);
}

void so_grammar_mask(const so_trie* t, int32_t width, const int32_t* eos, int32_t n_eos,
                     int32_t n_states, const int32_t* next, const uint8_t* flags, int32_t key,
                     uint32_t* out_words) {
  const int32_t words = (width + 31) / 32;
  memset(out_words, 0, sizeof(uint32_t) * (size_t)words);
  if (key == -1) {
    for (int32_t i = 0; i < width; ++i) set_bit(out_words, i, width);
    return;
  }
  if (key < -1) {
    set_bit(out_words, -2 - key, width);
    return;
  }
  if (key >= n_states) return;
  if (flags[key] & 2) walk(t, key, next, width, out_words);       /* consuming (:81) */
  if (flags[key] & 1)                                              /* accepting (:82) */
    for (int32_t e = 0; e < n_eos; ++e) set_bit(out_words, eos[e], width);
}

int32_t so_grammar_advance_bytes(int32_t s, const uint8_t* b, uint32_t len,
                                 const int32_t* next) {
  int32_t st = s;
  for (uint32_t i = 0; i < len; ++i) {
    st = next[(int64_t)st * 256 + b[i]];
    if (st < 0) return -1;
  }
  return st;
}

void so_grammar_verify_keys(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                            int32_t n_states, const int32_t* next, const int32_t* state,
                            int32_t B, const int32_t* tokens, int32_t k, int32_t* keys_out) {
  for (int32_t b = 0; b < B; ++b) {
    int32_t s = state[b];
    int32_t* o = keys_out + (int64_t)b * (k + 1);
    o[0] = s;
    for (int32_t i = 0; i < k; ++i) {
      /* step only a live grammar state (RequestConstraint.swift:98-99,139-143); once a
         step dies, the row and all later rows are free */
      if (s >= 0 && s < n_states) {
        const int32_t d = tokens[(int64_t)b * k + i];
        if (d >= 0 && d < count)
          s = so_grammar_advance_bytes(s, bytes + offsets[d], offsets[d + 1] - offsets[d], next);
      }
      o[i + 1] = s;
    }
  }
}

/* RequestConstraint.key (RequestConstraint.swift:85-92): in the thinking phase, free until
 * the budget is spent, then forced(closeId); afterwards the grammar state while it lives,
 * free once it is dead (or there is no grammar). */
static int32_t so_rq_key(const so_request_state* s) {
  if (s->in_think)
    return (s->budget >= 0 && s->close_id >= 0 && s->count >= s->budget) ? -2 - s->close_id : -1;
  return s->g >= 0 ? s->g : -1;
}

/* RequestConstraint.step (RequestConstraint.swift:94-102) */
static so_request_state so_rq_step(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                                   int32_t n_states, const int32_t* next, so_request_state s,
                                   int32_t t) {
  if (s.in_think) {
    if (t == s.close_id) s.in_think = 0;
    else s.count += 1;
  } else if (s.g >= 0 && s.g < n_states && t >= 0 && t < count) {
    s.g = so_grammar_advance_bytes(s.g, bytes + offsets[t], offsets[t + 1] - offsets[t], next);
  }
  return s;
}

static int so_rq_died(const so_request_state* prev, const so_request_state* nx) {
  return !prev->in_think && prev->g >= 0 && nx->g < 0;
}

void so_request_keys(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                     int32_t n_states, const int32_t* next, const so_request_state* states,
                     int32_t B, const int32_t* drafts, int32_t k, int32_t* keys_out) {
  for (int32_t b = 0; b < B; ++b) {
    so_request_state s = states[b];
    int32_t* o = keys_out + (int64_t)b * (k + 1);
    o[0] = so_rq_key(&s);
    int live = 1;
    for (int32_t i = 0; i < k; ++i) {
      if (live) {
        so_request_state prev = s;
        s = so_rq_step(count, offsets, bytes, n_states, next, s, drafts[(int64_t)b * k + i]);
        if (so_rq_died(&prev, &s)) live = 0;
      }
      o[i + 1] = live ? so_rq_key(&s) : -1;
    }
  }
}

void so_request_advance(int32_t count, const uint32_t* offsets, const uint8_t* bytes,
                        int32_t n_states, const int32_t* next, so_request_state* states,
                        int32_t B, const int32_t* drafts, int32_t k, const int32_t* accepted,
                        const int32_t* last) {
  for (int32_t b = 0; b < B; ++b) {
    so_request_state s = states[b];
    if (last[b] >= 0) {
      int32_t n = accepted ? accepted[b] : 0;
      n = n < 0 ? 0 : (n > k ? k : n);
      for (int32_t i = 0; i <= n; ++i) {
        const int32_t t = i < n ? drafts[(int64_t)b * k + i] : last[b];
        so_request_state nx = so_rq_step(count, offsets, bytes, n_states, next, s, t);
        const int died = so_rq_died(&s, &nx);
        s = nx;
        if (died) s.violated = 1;
      }
    }
    states[b] = s;
  }
}
