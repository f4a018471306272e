// Block bookkeeping of a shared KV pool (host), after lua/lgml/kvpool.lua.
//
// A pool of n blocks of `size` cells; blocks below cap are usable. A block
// has a reference count; a full block can carry a key (sha256 of the key of
// the block before it and its tokens, kvpool.lua:51-59); a keyed block with
// no reference stays cached until take() finds no free block and evict()
// hands it out (lowest priority, then least recently used, then deepest).
//
// All state lives in one caller-provided buffer of lgmlh_kvpool_bytes()
// (no allocation): a header, a fixed record per block, and an open-address
// table from key digests to blocks. Keys are 64 lowercase hex digits as the
// reference makes them; parent keys of first blocks may be any root string
// (stored as the sha256 digest of the string, so equal roots compare equal).
#include <string.h>

#include "common.h"

namespace lgmlh {
void sha256(const void *data, size_t n, uint8_t out[32]);
void sha256_hex(const void *data, size_t n, char out[65]);
}  // namespace lgmlh

using namespace lgmlh;

namespace {

constexpr uint32_t MAGIC = 0x6b76706cu;  // "kvpl"
constexpr int32_t EMPTY = -1, TOMB = -2;

struct Header {
  uint32_t magic;
  int32_t n, size, cap, used, low, cached;
  int32_t table;  // slots of the key table (power of 2)
  int64_t tick, evicted;
};

enum : uint8_t { F_KEY = 1, F_PART = 2 };

struct Block {
  int32_t refs;
  int32_t prio;
  int32_t depth;
  int32_t ntok;
  int64_t used;
  uint8_t flags, pad[7];
  uint8_t key[32];
  uint8_t parent[32];
  // int32_t tokens[size] follow
};

inline size_t block_bytes(int32_t size) {
  return (sizeof(Block) + 4 * (size_t)size + 7) & ~size_t(7);
}

inline int32_t table_slots(int32_t n) {
  int32_t t = 16;
  while (t < 2 * n) t <<= 1;
  return t;
}

struct View {
  Header *h;
  char *blocks;
  int32_t *tab;
  Block *blk(int32_t b) const { return (Block *)(blocks + (size_t)b * block_bytes(h->size)); }
  int32_t *toks(int32_t b) const { return (int32_t *)((char *)blk(b) + sizeof(Block)); }
};

bool view_of(void *mem, View &v) {
  if (!mem) return false;
  v.h = (Header *)mem;
  if (v.h->magic != MAGIC) return false;
  v.blocks = (char *)mem + ((sizeof(Header) + 63) & ~size_t(63));
  v.tab = (int32_t *)(v.blocks + (size_t)v.h->n * block_bytes(v.h->size));
  return true;
}

int hexval(char c) {
  if (c >= '0' && c <= '9') return c - '0';
  if (c >= 'a' && c <= 'f') return c - 'a' + 10;
  return -1;
}

// A key's 32-byte id: a 64-hex-digit key decodes; any other string (a root
// key) is hashed.
void key_id(const char *s, uint8_t out[32]) {
  size_t n = strlen(s);
  if (n == 64) {
    bool ok = true;
    for (int i = 0; i < 32 && ok; i++) {
      int a = hexval(s[2 * i]), b = hexval(s[2 * i + 1]);
      if (a < 0 || b < 0) ok = false;
      out[i] = (uint8_t)(a * 16 + b);
    }
    if (ok) return;
  }
  sha256(s, n, out);
  out[0] ^= 0x80;  // keep hashed roots apart from decoded keys
}

uint32_t slot0(const uint8_t id[32], int32_t t) {
  uint32_t x;
  memcpy(&x, id, 4);
  return x & (uint32_t)(t - 1);
}

int32_t tab_find(const View &v, const uint8_t id[32]) {
  int32_t t = v.h->table;
  for (uint32_t i = slot0(id, t), k = 0; k < (uint32_t)t; k++, i = (i + 1) & (t - 1)) {
    int32_t b = v.tab[i];
    if (b == EMPTY) return -1;
    if (b >= 0 && memcmp(v.blk(b)->key, id, 32) == 0) return (int32_t)i;
  }
  return -1;
}

void tab_insert(const View &v, const uint8_t id[32], int32_t b) {
  int32_t t = v.h->table;
  for (uint32_t i = slot0(id, t), k = 0; k < (uint32_t)t; k++, i = (i + 1) & (t - 1)) {
    if (v.tab[i] == EMPTY || v.tab[i] == TOMB) {
      v.tab[i] = b;
      return;
    }
  }
}

int32_t take_at(const View &v, int32_t b) {  // kvpool.lua:84-91
  v.blk(b)->refs = 1;
  v.h->used++;
  if (b == v.h->low) v.h->low = b + 1;
  return b;
}

void unkey(const View &v, int32_t b) {  // kvpool.lua:119-133
  Block *k = v.blk(b);
  if (k->flags & F_KEY) {
    int32_t s = tab_find(v, k->key);
    if (s >= 0 && v.tab[s] == b) v.tab[s] = TOMB;
  }
  k->flags = 0;
}

bool is_free(const View &v, int32_t b) { return v.blk(b)->refs == 0 && v.blk(b)->flags == 0; }

}  // namespace

extern "C" size_t lgmlh_kvpool_bytes(int32_t blocks, int32_t size) {
  if (blocks <= 0 || size <= 0) return 0;
  return ((sizeof(Header) + 63) & ~size_t(63)) + (size_t)blocks * block_bytes(size) +
         4 * (size_t)table_slots(blocks);
}

extern "C" int lgmlh_kvpool_init(void *mem, size_t bytes, int32_t blocks, int32_t size,
                                 int32_t cap) {
  if (!mem || blocks <= 0 || size <= 0 || cap < 0 || cap > blocks ||
      bytes < lgmlh_kvpool_bytes(blocks, size)) {
    set_error("kvpool_init: bad arguments");
    return LGMLH_EINVAL;
  }
  memset(mem, 0, lgmlh_kvpool_bytes(blocks, size));
  Header *h = (Header *)mem;
  h->magic = MAGIC;
  h->n = blocks;
  h->size = size;
  h->cap = cap;
  h->table = table_slots(blocks);
  View v;
  view_of(mem, v);
  for (int32_t i = 0; i < h->table; i++) v.tab[i] = EMPTY;
  return LGMLH_OK;
}

// kvpool.lua:102-116
extern "C" int32_t lgmlh_kvpool_take(void *pool, int32_t min) {
  View v;
  if (!view_of(pool, v)) return -1;
  int32_t from = v.h->low > min ? v.h->low : min;
  for (int32_t b = from; b < v.h->cap; b++)
    if (is_free(v, b)) return take_at(v, b);
  int32_t hi = from < v.h->cap ? from : v.h->cap;
  for (int32_t b = v.h->low; b < hi; b++)
    if (is_free(v, b)) return take_at(v, b);
  v.h->low = v.h->cap;
  return -1;
}

// kvpool.lua:139-160. Lua's pairs() visits blocks in no fixed order; this
// scan goes by block id, so an exact tie of (prio, used, depth) goes to the
// lowest id.
static int32_t victim_of(const View &v) {
  int32_t best = -1;
  for (int32_t b = 0; b < v.h->cap; b++) {
    Block *k = v.blk(b);
    if (!k->flags || k->refs) continue;
    if (best < 0) {
      best = b;
      continue;
    }
    Block *o = v.blk(best);
    if (k->prio < o->prio ||
        (k->prio == o->prio && (k->used < o->used || (k->used == o->used && k->depth > o->depth))))
      best = b;
  }
  return best;
}

// The block the next evict takes and its priority, with nothing changed:
// the moment of kvpool.lua:149-152, where the owner of the tensors copies a
// keyed block's cells out (on_evict) before the block loses its key.
extern "C" int32_t lgmlh_kvpool_victim(void *pool, int32_t *prio) {
  View v;
  if (!view_of(pool, v)) return -1;
  const int32_t b = victim_of(v);
  if (b >= 0 && prio) *prio = v.blk(b)->prio;
  return b;
}

extern "C" int32_t lgmlh_kvpool_evict(void *pool) {
  View v;
  if (!view_of(pool, v)) return -1;
  const int32_t best = victim_of(v);
  if (best < 0) return -1;
  unkey(v, best);
  v.h->cached--;
  v.h->evicted++;
  v.blk(best)->refs = 1;
  v.h->used++;
  return best;
}

// kvpool.lua:165-178
extern "C" int lgmlh_kvpool_ref(void *pool, int32_t b, int prio) {
  View v;
  if (!view_of(pool, v) || b < 0 || b >= v.h->n) {
    set_error("kvpool_ref: bad block");
    return LGMLH_EINVAL;
  }
  Block *k = v.blk(b);
  if (k->refs == 0) {
    if (!k->flags) {
      set_error("kvpool: ref of a free block");
      return LGMLH_EINVAL;
    }
    v.h->cached--;
    v.h->used++;
  }
  k->refs++;
  if (k->flags && prio > k->prio) k->prio = prio;
  return LGMLH_OK;
}

// kvpool.lua:183-198
extern "C" int lgmlh_kvpool_unref(void *pool, int32_t b) {
  View v;
  if (!view_of(pool, v) || b < 0 || b >= v.h->n || v.blk(b)->refs <= 0) {
    set_error("kvpool: unref of a free block");
    return LGMLH_EINVAL;
  }
  Block *k = v.blk(b);
  if (--k->refs > 0) return LGMLH_OK;
  v.h->used--;
  if (k->flags) {
    v.h->tick++;
    k->used = v.h->tick;
    v.h->cached++;
  } else if (b < v.h->low) {
    v.h->low = b;
  }
  return LGMLH_OK;
}

extern "C" int32_t lgmlh_kvpool_refs_of(void *pool, int32_t b) {
  View v;
  if (!view_of(pool, v) || b < 0 || b >= v.h->n) return 0;
  return v.blk(b)->refs;
}

static int put_info(const View &v, int32_t b, const char *parent, int32_t depth,
                    const int32_t *tokens, int32_t n, int prio) {
  Block *k = v.blk(b);
  key_id(parent, k->parent);
  k->depth = depth;
  k->ntok = n < v.h->size ? n : v.h->size;
  if (k->ntok > 0) memcpy(v.toks(b), tokens, 4 * (size_t)k->ntok);
  k->used = v.h->tick;
  k->prio = prio;
  return 1;
}

// kvpool.lua:217-226. Returns 1 when b got the key, 0 otherwise.
extern "C" int lgmlh_kvpool_publish(void *pool, int32_t b, const char *key, const char *parent,
                                    int32_t depth, const int32_t *tokens, int32_t n, int prio) {
  View v;
  if (!view_of(pool, v) || b < 0 || b >= v.h->n || !key || !parent || n < 0 ||
      (n > 0 && !tokens)) {
    set_error("kvpool_publish: bad arguments");
    return LGMLH_EINVAL;
  }
  uint8_t id[32];
  key_id(key, id);
  if (v.blk(b)->flags || tab_find(v, id) >= 0) return 0;
  Block *k = v.blk(b);
  memcpy(k->key, id, 32);
  k->flags = F_KEY;
  tab_insert(v, id, b);
  return put_info(v, b, parent, depth, tokens, n, prio);
}

// kvpool.lua:239-249: a partial block kept for longest_kid, no key.
extern "C" int lgmlh_kvpool_publish_part(void *pool, int32_t b, const char *parent,
                                         int32_t depth, const int32_t *tokens, int32_t n,
                                         int prio) {
  View v;
  if (!view_of(pool, v) || b < 0 || b >= v.h->n || !parent || n < 0 || (n > 0 && !tokens)) {
    set_error("kvpool_publish_part: bad arguments");
    return LGMLH_EINVAL;
  }
  if (v.blk(b)->flags || n == 0) return 0;
  v.blk(b)->flags = F_PART;
  memset(v.blk(b)->key, 0, 32);
  return put_info(v, b, parent, depth, tokens, n, prio);
}

// 0: no key; 1: a key (written as hex to out, 65 bytes); 2: the "part" marker.
extern "C" int lgmlh_kvpool_key_of(void *pool, int32_t b, char *out) {
  View v;
  if (!view_of(pool, v) || b < 0 || b >= v.h->n) return 0;
  Block *k = v.blk(b);
  if (k->flags & F_PART) return 2;
  if (!(k->flags & F_KEY)) return 0;
  if (out) {
    static const char hx[] = "0123456789abcdef";
    for (int i = 0; i < 32; i++) {
      out[2 * i] = hx[k->key[i] >> 4];
      out[2 * i + 1] = hx[k->key[i] & 15];
    }
    out[64] = 0;
  }
  return 1;
}

// kvpool.lua:261-263
extern "C" int32_t lgmlh_kvpool_lookup(void *pool, const char *key) {
  View v;
  if (!view_of(pool, v) || !key) return -1;
  uint8_t id[32];
  key_id(key, id);
  int32_t s = tab_find(v, id);
  return s < 0 ? -1 : v.tab[s];
}

// kvpool.lua:273-285: the kept block after parent that shares the longest
// prefix with tokens[0..max); ties go to the lowest block id.
extern "C" int32_t lgmlh_kvpool_longest_kid(void *pool, const char *parent, const int32_t *tokens,
                                            int32_t max, int32_t *shared) {
  View v;
  if (shared) *shared = 0;
  if (!view_of(pool, v) || !parent || max < 0 || (max > 0 && !tokens)) return -1;
  uint8_t id[32];
  key_id(parent, id);
  int32_t best = -1, bn = 0;
  for (int32_t b = 0; b < v.h->n; b++) {
    Block *k = v.blk(b);
    if (!k->flags || memcmp(k->parent, id, 32) != 0) continue;
    int32_t n = 0;
    const int32_t *t = v.toks(b);
    while (n < max && n < k->ntok && t[n] == tokens[n]) n++;
    if (n > bn) {
      best = b;
      bn = n;
    }
  }
  if (shared) *shared = bn;
  return best;
}

// kvpool.lua:289-293
extern "C" int lgmlh_kvpool_set_cap(void *pool, int32_t cap) {
  View v;
  if (!view_of(pool, v) || cap < 0 || cap > v.h->n) {
    set_error("kvpool: cap past the pool");
    return LGMLH_EINVAL;
  }
  v.h->cap = cap;
  if (v.h->low > cap) v.h->low = cap;
  return LGMLH_OK;
}

// out: n, size, cap, used, low, cached, tick, evicted
extern "C" int lgmlh_kvpool_stats(void *pool, int64_t *out) {
  View v;
  if (!view_of(pool, v) || !out) {
    set_error("kvpool_stats: bad arguments");
    return LGMLH_EINVAL;
  }
  out[0] = v.h->n;
  out[1] = v.h->size;
  out[2] = v.h->cap;
  out[3] = v.h->used;
  out[4] = v.h->low;
  out[5] = v.h->cached;
  out[6] = v.h->tick;
  out[7] = v.h->evicted;
  return LGMLH_OK;
}

// kvpool.lua:51-59: sha256 hex of parent "," tokens[0] "," ... tokens[n-1].
extern "C" int lgmlh_block_key(const char *parent, const int32_t *tokens, int32_t n, char *out) {
  if (!parent || !out || n < 0 || (n > 0 && !tokens)) {
    set_error("block_key: bad arguments");
    return LGMLH_EINVAL;
  }
  size_t pl = strlen(parent);
  size_t cap = pl + (size_t)n * 12 + 1;
  char stackbuf[4096];
  char *buf = cap <= sizeof stackbuf ? stackbuf : nullptr;
  if (!buf) {
    set_error("block_key: too many tokens for one block (%d)", n);
    return LGMLH_EINVAL;
  }
  memcpy(buf, parent, pl);
  size_t o = pl;
  for (int32_t i = 0; i < n; i++) {
    buf[o++] = ',';
    char tmp[16];
    int64_t x = tokens[i];
    int neg = x < 0;
    if (neg) x = -x;
    int t = 0;
    do {
      tmp[t++] = (char)('0' + x % 10);
      x /= 10;
    } while (x);
    if (neg) buf[o++] = '-';
    while (t) buf[o++] = tmp[--t];
  }
  sha256_hex(buf, o, out);
  return LGMLH_OK;
}
