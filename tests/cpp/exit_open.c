/* A C caller of libfa_rocm.so that exits with its context and an encoder
 * model still open (no fa_gemma_destroy, no fa_destroy).
 *
 * Regression program: a process that exits with a model open used to abort
 * in the HIP runtime's own teardown ("terminate called after throwing an
 * instance of 'std::bad_variant_access'"). The library now closes what is
 * still open from an exit handler registered at fa_create, before the
 * runtime tears itself down. Run by tests/test_gpu_exit.py, which expects
 * exit status 0 and no "terminate called" in the output. Plain C: the C ABI
 * alone, as a cgo or C caller uses it. */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "fa_rocm.h"
#include "fa_synth.h"

static int check(fa_ctx* ctx, int rc, const char* what) {
  if (rc != FA_OK) {
    fprintf(stderr, "%s: %s\n", what, fa_last_error(ctx));
    exit(2);
  }
  return rc;
}

static void set_mat(fa_model* m, fa_ctx* ctx, const char* name, int64_t out, int64_t in) {
  uint16_t* w = (uint16_t*)malloc((size_t)(out * in) * 2);
  int64_t shape[2] = {out, in};
  fa_synth_normal_bf16(99, name, 0.02, out * in, w);
  check(ctx, fa_gemma_set_weight(m, name, FA_DT_BF16, shape, 2, w), name);
  free(w);
}

static void set_norm(fa_model* m, fa_ctx* ctx, const char* name, int64_t n) {
  float* w = (float*)malloc((size_t)n * 4);
  fa_synth_normal_f32(99, name, 0.1, n, w);
  check(ctx, fa_gemma_set_weight(m, name, FA_DT_F32, &n, 1, w), name);
  free(w);
}

int main(void) {
  fa_ctx* ctx = NULL;
  if (fa_create(0, &ctx) != FA_OK) {
    fprintf(stderr, "fa_create: %s\n", fa_last_error(NULL));
    return 2;
  }
  fa_gemma_config c;
  memset(&c, 0, sizeof c);
  c.hidden_size = 768; c.num_hidden_layers = 2; c.num_attention_heads = 3; c.num_key_value_heads = 1;
  c.head_dim = 256; c.intermediate_size = 1152; c.vocab_size = 4096; c.sliding_window = 512;
  c.use_bidirectional = 1; c.sliding_window_pattern = 2; c.rope_local_base_freq = 1e4; c.rope_theta = 1e6;
  c.query_pre_attn_scalar = 256; c.rms_norm_eps = 1e-6f; c.max_tokens = 512;
  c.n_dense = 2; c.dense_out[0] = 3072; c.dense_out[1] = 768;
  fa_model* m = NULL;
  check(ctx, fa_gemma_create(ctx, &c, &m), "fa_gemma_create");
  set_mat(m, ctx, "embed_tokens.weight", 4096, 768);
  char name[128];
  for (int l = 0; l < 2; l++) {
    const char* norms[] = {"input_layernorm", "post_attention_layernorm", "pre_feedforward_layernorm",
                           "post_feedforward_layernorm"};
    for (int i = 0; i < 4; i++) {
      snprintf(name, sizeof name, "layers.%d.%s.weight", l, norms[i]);
      set_norm(m, ctx, name, 768);
    }
    snprintf(name, sizeof name, "layers.%d.self_attn.q_norm.weight", l); set_norm(m, ctx, name, 256);
    snprintf(name, sizeof name, "layers.%d.self_attn.k_norm.weight", l); set_norm(m, ctx, name, 256);
    snprintf(name, sizeof name, "layers.%d.self_attn.q_proj.weight", l); set_mat(m, ctx, name, 768, 768);
    snprintf(name, sizeof name, "layers.%d.self_attn.k_proj.weight", l); set_mat(m, ctx, name, 256, 768);
    snprintf(name, sizeof name, "layers.%d.self_attn.v_proj.weight", l); set_mat(m, ctx, name, 256, 768);
    snprintf(name, sizeof name, "layers.%d.self_attn.o_proj.weight", l); set_mat(m, ctx, name, 768, 768);
    snprintf(name, sizeof name, "layers.%d.mlp.gate_proj.weight", l); set_mat(m, ctx, name, 1152, 768);
    snprintf(name, sizeof name, "layers.%d.mlp.up_proj.weight", l); set_mat(m, ctx, name, 1152, 768);
    snprintf(name, sizeof name, "layers.%d.mlp.down_proj.weight", l); set_mat(m, ctx, name, 768, 1152);
  }
  set_norm(m, ctx, "norm.weight", 768);
  set_mat(m, ctx, "dense.0.linear.weight", 3072, 768);
  set_mat(m, ctx, "dense.1.linear.weight", 768, 3072);
  check(ctx, fa_gemma_finalize(m), "fa_gemma_finalize");
  int32_t ids[2 * 40];
  for (int i = 0; i < 80; i++) ids[i] = 7 + i;
  ids[0] = ids[40] = 2;
  const int32_t lengths[2] = {40, 25};
  float out[2 * 768];
  check(ctx, fa_gemma_embed_ids(m, ids, lengths, 2, 40, 0, out), "fa_gemma_embed_ids");
  double ss = 0;
  for (int i = 0; i < 768; i++) ss += (double)out[i] * out[i];
  printf("embedded 2 x 768, |e0|^2 = %.6f; exiting with the model and context open\n", ss);
  fflush(stdout);
  return 0;
}
