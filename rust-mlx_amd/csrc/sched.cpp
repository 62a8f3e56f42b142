// Cooperative equal-offset scheduler with a prefix cache (host side).
//
// Reference: batch::serve / admit / Row (src/bin/server/batch.rs:240-349,
// 28-140) and PrefixCache::get_or_prepare (src/speculative.rs:70-117):
//  * up to batch_size rows are active; queued jobs are admitted in arrival
//    order while a row is free;
//  * admission prepares the prompt (an exact-match LRU prefix cache of
//    prepared prompts, bounded by entry count and token budget) and emits the
//    greedy token of the prompt's last position;
//  * every step decodes, together, the active rows whose cache offset equals
//    the smallest offset among active rows (the laggards catch up, which
//    forms equal-offset groups);
//  * a row ends on a stop token (not emitted) or when it has emitted
//    max_tokens tokens; a prompt with prompt + max_tokens > max_context is
//    rejected.
// Caches are slots of the engine's arena: rows own one slot each, prefix
// entries own theirs, and a cache hit is a slot copy.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <deque>
#include <vector>

#include "../../include/mx355.h"

namespace {

struct Job {
  uint64_t id;
  std::vector<uint32_t> prompt;
  int32_t max_tokens;
  bool prefix;
};

struct Row {
  uint64_t id;
  int32_t slot;
  int64_t offset;  // positions in the slot's cache
  uint32_t next;   // token to feed at the next decode
  int32_t emitted;
  int32_t max_tokens;
  bool done;
};

struct Entry {
  std::vector<uint32_t> tokens;
  int32_t slot;
  uint32_t next;
};

}  // namespace

struct mx_sched {
  mx_sched_config cfg;
  mx_sched_backend be;
  std::deque<Job> queue;
  std::vector<Row> rows;
  std::deque<Entry> entries;  // LRU order: front = least recently used
  std::vector<bool> slot_used;

  int32_t take_slot() {
    for (size_t s = 0; s < slot_used.size(); ++s)
      if (!slot_used[s]) {
        slot_used[s] = true;
        return int32_t(s);
      }
    return -1;
  }
  void free_slot(int32_t s) {
    if (s >= 0 && size_t(s) < slot_used.size()) slot_used[s] = false;
  }
  bool is_stop(uint32_t t) const {
    for (int i = 0; i < cfg.n_stop; ++i)
      if (cfg.stop[i] == t) return true;
    return false;
  }
  size_t entry_tokens() const {
    size_t n = 0;
    for (const auto& e : entries) n += e.tokens.size();
    return n;
  }
};

namespace {

void push(std::vector<mx_sched_event>& ev, uint64_t job, uint32_t token, int32_t kind,
          int32_t detail) {
  ev.push_back(mx_sched_event{job, token, kind, detail});
}

// Row::emit: a stop token ends the row unemitted; otherwise the token is
// emitted and the row ends when it reaches max_tokens.
void emit(mx_sched& s, Row& r, uint32_t token, int32_t first_detail,
          std::vector<mx_sched_event>& ev) {
  if (s.is_stop(token)) {
    r.done = true;
    push(ev, r.id, token, MX_SCHED_STOP, 0);
    return;
  }
  r.next = token;
  r.emitted += 1;
  push(ev, r.id, token, MX_SCHED_TOKEN, first_detail);
  if (r.emitted == r.max_tokens) {
    r.done = true;
    push(ev, r.id, 0, MX_SCHED_LENGTH, 0);
  }
}

// Admission (Row::new + PrefixCache::get_or_prepare).  Returns false when no
// slot is free (the job stays queued).
bool admit(mx_sched& s, const Job& job, std::vector<mx_sched_event>& ev) {
  const int64_t len = int64_t(job.prompt.size());
  if (len == 0 || job.max_tokens < 1 || len + job.max_tokens > s.cfg.max_context) {
    push(ev, job.id, 0, MX_SCHED_ERROR, MX_EINVAL);
    return true;
  }
  int32_t slot = s.take_slot();
  if (slot < 0 && !s.entries.empty()) {  // a row may take a cache entry's slot
    s.free_slot(s.entries.front().slot);
    s.entries.pop_front();
    slot = s.take_slot();
  }
  if (slot < 0) return false;
  Row r{job.id, slot, len, 0, 0, job.max_tokens, false};
  uint32_t next = 0;
  bool hit = false;
  mx_status rc = MX_OK;
  if (job.prefix) {
    for (auto it = s.entries.begin(); it != s.entries.end(); ++it) {
      if (it->tokens == job.prompt) {
        Entry e = *it;
        s.entries.erase(it);
        rc = s.be.clone(s.be.ctx, e.slot, slot);
        next = e.next;
        s.entries.push_back(e);
        hit = true;
        break;
      }
    }
  }
  if (!hit && rc == MX_OK) {
    rc = s.be.prefill(s.be.ctx, slot, job.prompt.data(), int32_t(len), &next);
    if (rc == MX_OK && job.prefix && s.cfg.prefix_entries > 0 &&
        len <= int64_t(s.cfg.prefix_tokens)) {
      while (!s.entries.empty() &&
             (int32_t(s.entries.size()) >= s.cfg.prefix_entries ||
              s.entry_tokens() + size_t(len) > size_t(s.cfg.prefix_tokens))) {
        s.free_slot(s.entries.front().slot);
        s.entries.pop_front();
      }
      const int32_t es = s.take_slot();
      if (es >= 0) {
        if (s.be.clone(s.be.ctx, slot, es) == MX_OK) {
          s.entries.push_back(Entry{job.prompt, es, next});
        } else {
          s.free_slot(es);
        }
      }
    }
  }
  if (rc != MX_OK) {
    s.free_slot(slot);
    push(ev, job.id, 0, MX_SCHED_ERROR, rc);
    return true;
  }
  s.rows.push_back(r);
  emit(s, s.rows.back(), next, hit ? 1 : 0, ev);
  return true;
}

void retire(mx_sched& s) {
  std::vector<Row> keep;
  for (auto& r : s.rows) {
    if (r.done)
      s.free_slot(r.slot);
    else
      keep.push_back(r);
  }
  s.rows.swap(keep);
}

mx_status engine_prefill(void* ctx, int32_t slot, const uint32_t* tokens, int32_t count,
                         uint32_t* next) {
  mx_engine* e = static_cast<mx_engine*>(ctx);
  mx_status rc = mx_engine_reset_slot(e, slot);
  return rc == MX_OK ? mx_engine_prefill(e, slot, tokens, count, next) : rc;
}
mx_status engine_decode(void* ctx, const int32_t* slots, const uint32_t* tokens, int32_t rows,
                        uint32_t* next) {
  return mx_engine_decode_batch(static_cast<mx_engine*>(ctx), slots, tokens, rows, next);
}
mx_status engine_clone(void* ctx, int32_t src, int32_t dst) {
  return mx_engine_clone_slot(static_cast<mx_engine*>(ctx), src, dst);
}

}  // namespace

extern "C" {

__attribute__((visibility("default"))) mx_status mx_sched_create(const mx_sched_config* cfg,
                                                                  const mx_sched_backend* be,
                                                                  mx_sched** out) {
  if (!cfg || !be || !out || !be->prefill || !be->decode || !be->clone) return MX_EINVAL;
  if (cfg->batch_size < 1 || cfg->batch_size > 8 || cfg->slots < cfg->batch_size ||
      cfg->max_context < 2 || cfg->n_stop < 0 || cfg->n_stop > 8 || cfg->prefix_entries < 0 ||
      cfg->prefix_tokens < 0)
    return MX_EINVAL;
  mx_sched* s = new mx_sched();
  s->cfg = *cfg;
  s->be = *be;
  s->slot_used.assign(size_t(cfg->slots), false);
  *out = s;
  return MX_OK;
}

__attribute__((visibility("default"))) mx_status mx_sched_create_for_engine(
    mx_engine* e, const mx_sched_config* cfg, mx_sched** out) {
  if (!e) return MX_EINVAL;
  mx_sched_backend be{e, engine_prefill, engine_decode, engine_clone};
  return mx_sched_create(cfg, &be, out);
}

__attribute__((visibility("default"))) mx_status mx_sched_destroy(mx_sched* s) {
  delete s;
  return MX_OK;
}

__attribute__((visibility("default"))) mx_status mx_sched_submit(mx_sched* s, uint64_t job,
                                                                  const uint32_t* prompt,
                                                                  int32_t count,
                                                                  int32_t max_tokens,
                                                                  int32_t prefix_cache) {
  if (!s || count < 0 || (count > 0 && !prompt)) return MX_EINVAL;
  Job j{job, std::vector<uint32_t>(prompt, prompt + count), max_tokens, prefix_cache != 0};
  s->queue.push_back(std::move(j));
  return MX_OK;
}

__attribute__((visibility("default"))) mx_status mx_sched_cancel(mx_sched* s, uint64_t job) {
  if (!s) return MX_EINVAL;
  for (auto it = s->queue.begin(); it != s->queue.end(); ++it)
    if (it->id == job) {
      s->queue.erase(it);
      return MX_OK;
    }
  for (auto& r : s->rows)
    if (r.id == job && !r.done) {
      r.done = true;
      retire(*s);
      return MX_OK;
    }
  return MX_EINVAL;
}

__attribute__((visibility("default"))) mx_status mx_sched_step(mx_sched* s,
                                                                mx_sched_event* events,
                                                                int32_t capacity, int32_t* count,
                                                                int32_t* decoded_rows) {
  if (!s || !count || (capacity > 0 && !events)) return MX_EINVAL;
  if (capacity < 4 * s->cfg.batch_size) return MX_EINVAL;
  std::vector<mx_sched_event> ev;
  // admit queued jobs while a row is free
  while (!s->queue.empty() && int32_t(s->rows.size()) < s->cfg.batch_size) {
    if (!admit(*s, s->queue.front(), ev)) break;
    s->queue.pop_front();
  }
  retire(*s);
  int32_t decoded = 0;
  if (!s->rows.empty()) {
    int64_t off = s->rows.front().offset;
    for (const auto& r : s->rows) off = std::min(off, r.offset);
    std::vector<int32_t> idx, slots;
    std::vector<uint32_t> toks;
    for (size_t i = 0; i < s->rows.size(); ++i)
      if (s->rows[i].offset == off) {
        idx.push_back(int32_t(i));
        slots.push_back(s->rows[i].slot);
        toks.push_back(s->rows[i].next);
      }
    std::vector<uint32_t> next(idx.size(), 0);
    const mx_status rc = s->be.decode(s->be.ctx, slots.data(), toks.data(), int32_t(idx.size()),
                                      next.data());
    for (size_t g = 0; g < idx.size(); ++g) {
      Row& r = s->rows[size_t(idx[g])];
      if (rc != MX_OK) {
        r.done = true;
        push(ev, r.id, 0, MX_SCHED_ERROR, rc);
      } else {
        r.offset += 1;
        emit(*s, r, next[g], 0, ev);
      }
    }
    decoded = int32_t(idx.size());
    retire(*s);
  }
  if (int32_t(ev.size()) > capacity) return MX_EINVAL;  // cannot happen: <= 4 per row
  std::memcpy(events, ev.data(), ev.size() * sizeof(mx_sched_event));
  *count = int32_t(ev.size());
  if (decoded_rows) *decoded_rows = decoded;
  return MX_OK;
}

__attribute__((visibility("default"))) int32_t mx_sched_pending(const mx_sched* s) {
  return s ? int32_t(s->queue.size() + s->rows.size()) : 0;
}

__attribute__((visibility("default"))) int32_t mx_sched_cached(const mx_sched* s) {
  return s ? int32_t(s->entries.size()) : 0;
}

}  // extern "C"
