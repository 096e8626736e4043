/* ref_model.c -- expose the reference's config parsing and RoPE frequency
 * table for golden-vector generation.
 *
 * TEST INFRASTRUCTURE ONLY.  This file contains no reference code.  Like
 * ref_harness.c it is compiled by oracle/Makefile (target `ref`) with -I at
 * /root/reference/src, so the `#include "model_load.c"` below pulls in the
 * reference's src/model_load.c from where it lies, unmodified: the only way
 * to reach its `static` config_from_json (model_load.c:242-292) and
 * build_rope_inv_freq (model_load.c:299-325).  It links against the
 * reference's own vendor/cJSON.c, src/safetensors_loader.c and src/tensor.c;
 * the output goes only to oracle/_ref/ (git-ignored).
 */
#include "model_load.c"

/* Parse <model_dir>/config.json as the engine does and build its RoPE
 * inverse-frequency table.  ints[] receives qk_rope_head_dim,
 * rope_interleaved, q_lora_rank, n_heads, qk_nope_head_dim, kv_lora_rank,
 * v_head_dim, hidden_size; flts[] receives rms_eps, mla_norm_eps,
 * softmax_scale, rope_theta, rope_factor, rope_beta_fast, rope_beta_slow,
 * rope_orig_max.  inv must hold qk_rope_head_dim / 2 floats. */
int ref_config_rope(const char *model_dir, float *inv, int *ints, float *flts) {
    Config c = config_from_json(model_dir);
    float *f = build_rope_inv_freq(&c);
    memcpy(inv, f, (size_t)(c.qk_rope_head_dim / 2) * sizeof(float));
    free(f);
    const int iv[8] = {c.qk_rope_head_dim, c.rope_interleaved, c.q_lora_rank, c.n_heads,
                       c.qk_nope_head_dim, c.kv_lora_rank, c.v_head_dim, c.hidden_size};
    const float fv[8] = {c.rms_eps, c.mla_norm_eps, c.softmax_scale, c.rope_theta,
                         c.rope_factor, c.rope_beta_fast, c.rope_beta_slow, c.rope_orig_max};
    memcpy(ints, iv, sizeof(iv));
    memcpy(flts, fv, sizeof(fv));
    return 0;
}
