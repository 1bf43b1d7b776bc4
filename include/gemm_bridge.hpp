// gemm_bridge.hpp -- C++ mirror of the reference engine's GEMM operator layer,
// implemented over the C ABI in mi_gemm.h.
//
// Same names, argument meaning and error behaviour as the reference's
// metal_bridge GEMM entry points (cpp/include/gpu_kernel/MetalBridge.hpp) and
// Tensor::matmul (cpp/include/Tensor.hpp:230, cpp/src/Tensor.cpp:174-228), so an
// engine built on them can switch namespaces.  Differences, all deliberate:
//   * pointers are HIP device pointers (the reference wrapped unified-memory host
//     pointers, MetalBridge.mm:765-834);
//   * the reference's float* parameters of gemm_backward / gemm_proj_trans_b /
//     residual_add carry bf16 storage (buffers sized with sizeof(__bf16),
//     MetalBridge.mm:1353-1355,1928; residual_add.metal:15-17); the mirror keeps
//     that interpretation and adds explicit fp32 variants;
//   * errors print "[mi_bridge] <function>: <reason>" to stderr and return, as the
//     bridge did (MetalBridge.mm:1360); last_status() exposes the code.
#pragma once
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "mi_gemm.h"

namespace mi_bridge {

// MetalBridge.hpp:20-21
void initialize();
bool is_available();

// MetalBridge.hpp:29-30.  Inside a scope every call is enqueued on the bridge's
// stream without waiting; end_scope() waits once.  Outside a scope each call
// waits for its own completion (MetalBridge.mm:1384-1406).
void begin_scope();
void end_scope();
inline void start_batch() { begin_scope(); }
inline void commit_batch() { end_scope(); }

// The stream the bridge enqueues on (a hipStream_t), created on first use.
void* stream();

// Status of the last bridge call on this thread (mi_status).
int last_status();

// MetalBridge.hpp:39-42: C[M,N] = op(A) op(B), bf16 in / bf16 out, fp32 accumulate.
// is_forward is accepted and ignored, as in gemm_bf16.metal.
void gemm_bf16(const void* A, const void* B, void* C, size_t M, size_t N, size_t K,
               bool transA = false, bool transB = false, bool is_forward = false);

// MetalBridge.hpp:44-46: C = (SiLU(gate) * up) * B, bf16, gate/up [M,K], B [K,N].
void fused_swiglu_gemm(const void* gate_proj, const void* up_proj, const void* B, void* C,
                       size_t M, size_t N, size_t K);

// MetalBridge.hpp:119-120: C = SiLU(A*Bg) * (A*Bu), fp32, A [M,K], Bg/Bu [K,N].
void gemm_ffn(const float* a, const float* b_gate, const float* b_up, float* c, size_t M,
              size_t N, size_t K);

// MetalBridge.hpp:121: C = A*B, fp32 row-major NN (the cblas_sgemm call of
// MetalBridge.mm:695-697, here on the GPU).
void gemm_proj(const float* a, const float* b, float* c, size_t M, size_t N, size_t K);

// MetalBridge.hpp:122-123 / MetalBridge.mm:1925-1930: C[M,N] = A^T B with A
// stored [K,M], bf16 storage, overwriting C.
void gemm_backward(const float* a_transposed, const float* b, float* c, size_t M, size_t N,
                   size_t K);

// The engine's weight-gradient semantics (Transformer.cpp:236,288-289,
// gemm_backward.metal:104-115): dW[M,N] (fp32) += A^T B, A [K,M] and B [K,N] bf16.
void gemm_backward_accumulate(const void* a_transposed, const void* b, float* c, size_t M,
                              size_t N, size_t K);

// MetalBridge.hpp:124-125 / MetalBridge.mm:1932-1936: C = A B^T, B stored [N,K],
// bf16 storage.
void gemm_proj_trans_b(const float* a, const float* b_transposed, float* c, size_t M, size_t N,
                       size_t K);

// MetalBridge.hpp:49-51: causal GQA attention forward, bf16.  Q [B,nH,S,d], K/V
// [B,nKV,S,d], O [B,nH,S,d] (the output layout of flash_attn_fwd.metal); query
// head h reads KV head h / (nH/nKV).  head_dim 64 (the reference kernel's) and 128
// run the fused kernel; another head_dim below 128 and a multiple of 8 runs the next
// larger one on bridge-owned copies of Q, K, V whose columns past head_dim are zero,
// with the scale 1/sqrt(head_dim) (mi_flash_attn_fwd_scaled); any other head_dim runs the
// materialised form: S and P in a bridge-owned [B,nH,S,S] bf16 buffer, batched
// GEMMs and the softmax kernel.
void flash_attn_fwd(const void* Q, const void* K, const void* V, void* O, size_t batch,
                    size_t n_heads, size_t n_kv, size_t seq_len, size_t head_dim);

// MetalBridge.hpp:54-57: gradients of the causal GQA attention, bf16, dO and dQ
// [B,nH,S,d], dK/dV [B,nKV,S,d] summed over each KV group's query heads.  Like
// the reference kernel it takes no forward state: the forward's O and row
// log-sum-exp are recomputed into bridge-owned device buffers first.  head_dim 64
// and 128: the fused kernels; another head_dim below 128 (multiple of 8): the next
// larger fused kernels on zero-padded copies, as in flash_attn_fwd; any other
// head_dim: the materialised backward (P and dP in
// bridge-owned buffers).
void fused_attn_bwd(const void* Q, const void* K, const void* V, const void* dO, void* dQ,
                    void* dK, void* dV, size_t batch, size_t n_heads, size_t n_kv,
                    size_t seq_len, size_t head_dim);

// MetalBridge.hpp:89-91: fused softmax cross-entropy (cross_entropy.metal) over
// total_tokens rows of vocab_size bf16 logits.  grad_logits (fp32, device) receives
// (softmax - onehot) / total_tokens; *loss_out (host) the mean of
// -log(max(p_target, 1e-15)), written when the work has run: on return outside a
// scope, at end_scope() inside one (the reference's copy-back).  targets are device
// memory.
void cross_entropy(const void* logits, const uint32_t* targets, float* loss_out,
                   float* grad_logits, size_t total_tokens, size_t vocab_size);

// MetalBridge.hpp:60-61: y = x / sqrt(mean(x^2) + eps) * w per row of dims values,
// bf16 storage behind the float pointers (rms_norm_forward.metal; RMSNorm.cpp:48-75).
void rms_norm_forward(const float* input, float* output, const float* weight, float eps,
                      size_t num_rows, size_t dims);

// MetalBridge.hpp:62-64: dx and the weight gradient (written, as
// rms_norm_backward.metal does), bf16 storage (RMSNorm.cpp:77-180).  grad_weight may
// be NULL.  The weight-gradient workspace is bridge-owned.
void rms_norm_backward(const float* grad_output, const float* input, const float* weight,
                       float* grad_input, float* grad_weight, float eps, size_t num_rows,
                       size_t dims);

// MetalBridge.hpp:79-81: x_residual += residual; output = rmsnorm(x_residual) * weight,
// fp32 (fused_add_norm.metal; the decoder layer's h += out, ffn_in = norm(h),
// Transformer.cpp:150-158).
void fused_add_norm(float* x_residual, const float* residual, const float* weight, float* output,
                    size_t num_rows, size_t D, float eps);

// The decoder layer's norm and the projection that consumes it as one call
// (Transformer.cpp:147-162: fused_add_norm, then ffn_in.matmul(w_gate / w_up);
// Attention.cpp:196-201: x_norm.matmul(Wq / Wk / Wv)): x += residual (when given,
// in place, bf16), then out = rmsnorm(x) * W with the norm folded into the GEMM:
// 1/rms per row (mi_rmsnorm_fwd without y), W' = diag(norm_weight) W
// (mi_rmsnorm_fold_weight, bridge-owned), out = diag(1/rms) x W' (mi_gemm with
// epi->row_scale).  The normalised activations are never written.  x, residual, W
// [dims, N], out [rows, N] bf16; norm_weight fp32 [dims].  No counterpart in the
// reference: it replaces the pair of calls.
void fused_norm_matmul(void* x, const void* residual, const float* norm_weight, const void* W, void* out,
                       size_t rows, size_t dims, size_t N, float eps);

// MetalBridge.hpp:82-85: grad_input = rmsnorm_backward(grad_output, input) + residual,
// bf16 activations, fp32 weight (fused_backward_add_norm.metal, Transformer.cpp:441-466).
void fused_backward_add_norm(const void* grad_output, const void* input, const void* weight,
                             const void* residual, void* grad_input, size_t num_rows, size_t D,
                             float eps);

// MetalBridge.hpp:78: a[i] += b[i] on bf16 storage (residual_add.metal:15-28).
void residual_add(float* a, const float* b, size_t n);
// fp32 storage variant.
void residual_add_f32(float* a, const float* b, size_t n);

// ---- Tensor::matmul mirror ---------------------------------------------------

enum class DType : uint8_t { FP32, BF16 };  // Tensor.hpp:14

// A non-owning view of a row-major device tensor with up to 5 dims (Tensor.hpp:31-76).
struct DeviceTensor {
  void* data = nullptr;
  std::vector<size_t> shape;
  DType dtype = DType::BF16;
  size_t numel() const {
    size_t n = 1;
    for (size_t d : shape) n *= d;
    return n;
  }
  size_t itemsize() const { return dtype == DType::BF16 ? 2 : 4; }
};

// Shape of `a.matmul(b)` (Tensor.cpp:174-209), throwing std::invalid_argument with
// the reference's messages on rank < 2, inner or batch mismatch.
std::vector<size_t> matmul_shape(const DeviceTensor& a, const DeviceTensor& b);

// out = a.matmul(b): projection (N-D x 2-D) or same-rank batched product, one
// launch for all batch slices; out.dtype = a.dtype, out.data preallocated with
// matmul_shape(a, b) elements.  a and b must share a dtype.
void matmul(const DeviceTensor& a, const DeviceTensor& b, DeviceTensor& out);

// ---- checkpoint weights (Checkpoint.cpp) ---------------------------------------

// One entry of a safetensors header: dtype "F32" / "BF16" / "F16" (others are listed
// but not loadable), shape, and byte range within the payload.
struct TensorInfo {
  std::string name, dtype;
  std::vector<size_t> shape;
  size_t begin = 0, end = 0;
};

// A memory-mapped safetensors file (8-byte header length, JSON header, payload;
// Checkpoint.cpp:301-400).  open() checks the header (at most 10 MiB, as the
// reference) and that every tensor's byte range lies in the payload and matches its
// shape; on failure it returns false and error() says why.
class SafetensorsFile {
 public:
  SafetensorsFile() = default;
  ~SafetensorsFile();
  SafetensorsFile(const SafetensorsFile&) = delete;
  SafetensorsFile& operator=(const SafetensorsFile&) = delete;
  bool open(const std::string& path);
  void close();
  const std::string& error() const { return err_; }
  const std::vector<TensorInfo>& tensors() const { return tensors_; }
  const TensorInfo* find(const std::string& name) const;
  const uint8_t* data(const TensorInfo& t) const;  // host pointer into the mapping
  // A Python/MLX checkpoint holds "tok_embeddings.weight" (Checkpoint.cpp:404-406).
  bool is_python_format() const;

 private:
  uint8_t* map_ = nullptr;
  size_t size_ = 0, payload_ = 0;
  std::vector<TensorInfo> tensors_;
  std::string err_;
};

// Model dimensions (the reference's TransformerConfig fields the weights depend on).
struct ModelConfig {
  size_t n_layers = 0, hidden_dim = 0, n_heads = 0, n_kv_heads = 0, head_dim = 0;
  size_t intermediate_dim = 0, vocab_size = 0;
};

// Caller-allocated device buffers in the engine layout: Wq [H, nH*hd], Wk/Wv
// [H, nKV*hd], Wo [nH*hd, H], w_gate/w_up [H, I], w_down [I, H], norms [H],
// token_embeddings [V, H], output_projection [H, V]; all of `dtype`.
struct LayerWeights {
  void *attn_norm = nullptr, *ffn_norm = nullptr;
  void *Wq = nullptr, *Wk = nullptr, *Wv = nullptr, *Wo = nullptr;
  void *w_gate = nullptr, *w_up = nullptr, *w_down = nullptr;
};
struct ModelWeights {
  DType dtype = DType::BF16;
  void *token_embeddings = nullptr, *output_projection = nullptr, *final_norm = nullptr;
  std::vector<LayerWeights> layers;
};

// The model part of Checkpoint::load (Checkpoint.cpp:331-388, 532-570): reads a
// Python/MLX file (nn.Linear [out, in] matrices, fused wqkv and w12, transposed and
// cut into the engine's matrices) or an engine file (engine names and layout) into
// `w`, widening or rounding to w.dtype on the GPU.  Fails (false, message on stderr)
// on a bad file, a missing tensor or a shape mismatch.
bool load_weights(const std::string& path, const ModelConfig& cfg, const ModelWeights& w);

// ---- GEMM profiler (gemm_profiler.hpp:18-117) -------------------------------------

// One GEMM call: shape, transposes and its GPU time (HIP events around the call's
// kernels on the bridge stream; the reference recorded host-side encoding time,
// MetalBridge.mm:1408-1411), plus the plan that ran.
struct GemmRecord {
  size_t M, N, K;
  bool transA, transB;
  double elapsed_ms;
  std::string kernel;
  size_t batch = 1;
};

// Same methods as the reference's GemmProfiler singleton.  Recording is off until
// enable(); it covers every GEMM issued through this bridge or the C ABI.
class GemmProfiler {
 public:
  static GemmProfiler& instance();
  void enable(bool on = true);
  void begin_step();                            // drop the step's records
  std::vector<GemmRecord> records() const;      // waits for the recorded kernels
  void print_summary(double step_gpu_ms) const; // per (M,N,K,tA,tB): calls, GPU ms, TFLOP/s
  static const char* op_name(size_t M, size_t N, size_t K, bool tA, bool tB);

 private:
  GemmProfiler() = default;
};

// MetalBridge.hpp:141-145 (there extern variables; here functions, because the GPU
// times are read from events when asked for): GPU time and number of recorded GEMM
// calls since the last reset_profile_stats().
double accum_gpu_time_ms();
size_t count_gpu_calls();
void reset_profile_stats();

}  // namespace mi_bridge
