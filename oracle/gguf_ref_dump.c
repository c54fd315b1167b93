/*
 * gguf_ref_dump.c -- test infrastructure only: prints what the reference's
 * own GGUF reader (gguf.c, compiled where it lies into oracle/_ref) makes of
 * one or more shards, so the tests can compare the library's reader with
 * it on the same files.  Output, one record per line:
 *   types <id> <blck> <size> ...      (the ggml type table, for "types")
 *   shard <i> <version> <alignment> <data_start> <n_kv> <n_tensors>
 *   kv <i> <key> <type> <scalar-or-array-info>
 *   tensor <name> <type> <n_dims> <d0> <d1> <d2> <d3> <nbytes> <abs_offset> <shard>
 * Exit status 1 (and "error") when gguf_load_manifest rejects the files.
 */
#include <inttypes.h>
#include <stdio.h>
#include <string.h>

#include "gguf.h"

static void print_kv(int shard, const gguf_kv *kv) {
  printf("kv %d %s %d", shard, kv->key, (int)kv->type);
  switch (kv->type) {
    case GGUF_TYPE_UINT8: printf(" %u", kv->v.u8); break;
    case GGUF_TYPE_INT8: printf(" %d", kv->v.i8); break;
    case GGUF_TYPE_UINT16: printf(" %u", kv->v.u16); break;
    case GGUF_TYPE_INT16: printf(" %d", kv->v.i16); break;
    case GGUF_TYPE_UINT32: printf(" %u", kv->v.u32); break;
    case GGUF_TYPE_INT32: printf(" %d", kv->v.i32); break;
    case GGUF_TYPE_UINT64: printf(" %" PRIu64, kv->v.u64); break;
    case GGUF_TYPE_INT64: printf(" %" PRId64, kv->v.i64); break;
    case GGUF_TYPE_FLOAT32: printf(" %.9g", (double)kv->v.f32); break;
    case GGUF_TYPE_FLOAT64: printf(" %.17g", kv->v.f64); break;
    case GGUF_TYPE_BOOL: printf(" %d", kv->v.b ? 1 : 0); break;
    case GGUF_TYPE_STRING: printf(" %s", kv->v.str); break;
    case GGUF_TYPE_ARRAY: printf(" %d %" PRIu64, (int)kv->arr.elem_type, kv->arr.n); break;
    default: break;
  }
  printf("\n");
}

int main(int argc, char **argv) {
  if (argc >= 2 && strcmp(argv[1], "types") == 0) {
    printf("types");
    for (int t = 0; t < GGML_TYPE_COUNT; ++t)
      printf(" %d %zu %zu", t, ggml_blck_size((ggml_type)t), ggml_type_size((ggml_type)t));
    printf("\n");
    return 0;
  }
  if (argc < 2) {
    fprintf(stderr, "usage: %s types | shard.gguf [shard.gguf ...]\n", argv[0]);
    return 2;
  }
  gguf_manifest m;
  if (gguf_load_manifest(&m, (const char *const *)(argv + 1), argc - 1) != 0) {
    printf("error\n");
    return 1;
  }
  for (int i = 0; i < m.n_shards; ++i) {
    const gguf_shard *s = &m.shards[i];
    printf("shard %d %u %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 "\n", i, s->version, s->alignment,
           s->data_start, s->n_kv, s->n_tensors);
    for (uint64_t k = 0; k < s->n_kv; ++k) print_kv(i, &s->kvs[k]);
  }
  for (uint64_t k = 0; k < m.total_tensors; ++k) {
    const gguf_tensor *t = m.all_tensors[k];
    printf("tensor %s %d %u %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 " %" PRIu64 " %d\n", t->name,
           (int)t->type, t->n_dims, t->dims[0], t->n_dims > 1 ? t->dims[1] : 1, t->n_dims > 2 ? t->dims[2] : 1,
           t->n_dims > 3 ? t->dims[3] : 1, t->nbytes, t->abs_offset, t->shard_idx);
  }
  gguf_free_manifest(&m);
  return 0;
}
