/* Exported entry points over the reference's static CPU kernels. */
#undef cpu_swiglu
float ref_bf16_to_f32(uint16_t v) { return bf16_to_f32(v); }
uint16_t ref_f32_to_bf16(float f) { return f32_to_bf16(f); }
void ref_cpu_dequant_matvec(const uint32_t *W, const uint16_t *s, const uint16_t *b,
                            const float *x, float *out, int out_dim, int in_dim, int gs) {
    cpu_dequant_matvec(W, s, b, x, out, out_dim, in_dim, gs);
}
void ref_main_dequant_matvec_4bit(const uint32_t *W, const uint16_t *s, const uint16_t *b,
                                  const float *x, float *out, uint32_t out_dim,
                                  uint32_t in_dim, uint32_t gs) {
    cpu_dequant_matvec_4bit(W, s, b, x, out, out_dim, in_dim, gs);
}
void ref_cpu_swiglu(const float *g, const float *u, float *o, int dim) { cpu_swiglu(g, u, o, dim); }
void ref_main_swiglu(const float *g, const float *u, float *o, uint32_t dim) { main_m_cpu_swiglu(g, u, o, dim); }
float ref_cpu_sigmoid(float x) { return cpu_sigmoid(x); }
void ref_cpu_softmax(float *x, int dim) { cpu_softmax(x, dim); }
void ref_cpu_topk(const float *s, int dim, int K, int *idx, float *val) { cpu_topk(s, dim, K, idx, val); }
void ref_cpu_normalize_weights(float *w, int K) { cpu_normalize_weights(w, K); }
void ref_cpu_vec_madd(float *d, const float *s, float sc, int dim) { cpu_vec_madd(d, s, sc, dim); }
void ref_cpu_rms_norm(const float *x, const uint16_t *w, float *o, int dim, float eps) { cpu_rms_norm(x, w, o, dim, eps); }
