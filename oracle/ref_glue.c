/* ref_glue.c - test-only probe of two of QStream's engine helpers.
 *
 * Test infrastructure, never part of the product.  apply_rope
 * (src/engine.c:205-234) and kv_cache_store (src/engine.c:240-293) are
 * static in the reference's engine translation unit, so this file includes
 * that unit as it lies in the reference tree (oracle/Makefile compiles it
 * with the reference headers and strict fp) and exports a call of each.
 * The rest of engine.c's dependencies (model loader, tokenizer, sampler,
 * arena) are left unresolved: the library is loaded with lazy binding and
 * neither helper calls them.
 */
#include "engine.c"

/* apply_rope on q [n_heads][head_dim] and k [n_kv][head_dim], in place */
void ref_glue_apply_rope(float* q, float* k, int head_dim, int position, float theta, int n_heads,
                         int n_kv) {
    apply_rope(q, k, head_dim, position, theta, n_heads, n_kv);
}

/* kv_cache_store of row `position` into one layer's caches laid out as
 * [n_kv][max_seq][head_dim] int8 and [n_kv][max_seq] scales */
void ref_glue_kv_store(int8_t* kc, int8_t* vc, float* ks, float* vs, int max_seq, int n_kv, int head_dim,
                       int position, const float* k, const float* v) {
    QSFKVHead heads[64];
    QSFKVCache kv;
    memset(&kv, 0, sizeof kv);
    if (n_kv > 64) return;
    for (int h = 0; h < n_kv; h++) {
        heads[h].k_cache = kc + (size_t)h * max_seq * head_dim;
        heads[h].v_cache = vc + (size_t)h * max_seq * head_dim;
        heads[h].k_scales = ks + (size_t)h * max_seq;
        heads[h].v_scales = vs + (size_t)h * max_seq;
    }
    kv.heads = heads;
    kv.num_layers = 1;
    kv.num_kv_heads = n_kv;
    kv.head_dim = head_dim;
    kv.max_seq = max_seq;
    kv_cache_store(&kv, 0, position, k, v);
}
