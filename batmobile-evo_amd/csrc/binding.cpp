// _batmobile: PyTorch-ROCm extension module over libbatmobile_hip.so.
//
// Replaces reference python/bindings.cpp (module `_batmobile`, :597-811): same
// function names, argument names, defaults, argument checks (TORCH_CHECK ->
// Python RuntimeError), output allocation (torch::empty on the input's device)
// and stream (the caller's current stream).  Host code only: every launch goes
// through the C ABI declared in include/batmobile_hip.h.
//
// Extensions beyond the reference surface (documented per function below):
// spherical_harmonics_normalized(+_backward), sh_tp_scatter and neighbor_list.
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <cstdint>
#include <string>
#include <tuple>

#include "batmobile_hip.h"

namespace {

void check_device(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
    TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
}

// Stream of the tensor's device; checks the tensor first, so a CPU tensor gives
// the argument error before any HIP call is made.
hipStream_t current_stream(const torch::Tensor& t) {
    TORCH_CHECK(t.is_cuda(), "inputs must be CUDA tensors");
    return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

template <typename T>
const T* cptr(const torch::Tensor& t, const char* name) {
    check_device(t, name);
    return t.data_ptr<T>();
}
template <typename T>
T* mptr(torch::Tensor& t, const char* name) {
    check_device(t, name);
    return t.data_ptr<T>();
}

void check_status(int rc, const char* what) {
    if (rc == BATMOBILE_HIP_OK) return;
    if (rc == BATMOBILE_HIP_ERR_ARG) TORCH_CHECK(false, what, ": invalid argument");
    if (rc == BATMOBILE_HIP_ERR_WORKSPACE) TORCH_CHECK(false, what, ": workspace too small");
    if (rc == BATMOBILE_HIP_ERR_SCRATCH) TORCH_CHECK(false, what, ": larger than the static scratch");
    TORCH_CHECK(false, "HIP error in ", what, ": ", hipGetErrorString(static_cast<hipError_t>(rc)));
}

// 16-byte aligned contiguous view (the MFMA kernels read float4 rows).
torch::Tensor aligned16(const torch::Tensor& t) {
    if ((reinterpret_cast<uintptr_t>(t.data_ptr()) & 15) == 0) return t;
    return t.clone(at::MemoryFormat::Contiguous);
}

torch::TensorOptions f32_like(const torch::Tensor& t) {
    return torch::TensorOptions().dtype(torch::kFloat32).device(t.device());
}

// ---------------------------------------------------------------------------
// spherical harmonics (reference bindings.cpp:43-114, 236-280)
// ---------------------------------------------------------------------------
void check_vectors(const torch::Tensor& v) {
    TORCH_CHECK(v.dim() == 2, "edge_vectors must be 2D");
    TORCH_CHECK(v.size(1) == 3, "edge_vectors must have shape [N, 3]");
    TORCH_CHECK(v.dtype() == torch::kFloat32, "edge_vectors must be float32");
}

torch::Tensor sh_impl(const torch::Tensor& v, int64_t L_max, int normalize) {
    check_vectors(v);
    TORCH_CHECK(L_max >= 0 && L_max <= 6, "L_max must be in [0, 6]");
    const int64_t N = v.size(0);
    torch::Tensor Y = torch::empty({N, (L_max + 1) * (L_max + 1)}, f32_like(v));
    if (N == 0) return Y;
    const c10::DeviceGuard guard(v.device());
    check_status(batteries_spherical_harmonics(cptr<float>(v, "edge_vectors"),
                                               mptr<float>(Y, "Y_lm"), N, (int)L_max, normalize,
                                               current_stream(v)),
                 "spherical_harmonics");
    return Y;
}

torch::Tensor spherical_harmonics(const torch::Tensor& edge_vectors, int64_t L_max) {
    return sh_impl(edge_vectors, L_max, 0);
}

// Extension: SH of v / max(|v|, 1e-10) in one pass (the normalisation of
// reference python/batmobile/autograd.py:46-58 fused into the kernel).
torch::Tensor spherical_harmonics_normalized(const torch::Tensor& edge_vectors, int64_t L_max) {
    return sh_impl(edge_vectors, L_max, 1);
}

void spherical_harmonics_inplace(const torch::Tensor& edge_vectors, torch::Tensor& Y_lm,
                                 int64_t L_max) {
    check_vectors(edge_vectors);
    TORCH_CHECK(L_max >= 0 && L_max <= 6, "L_max must be in [0, 6]");
    const int64_t N = edge_vectors.size(0);
    const int64_t K = (L_max + 1) * (L_max + 1);
    TORCH_CHECK(Y_lm.dim() == 2, "Y_lm must be 2D");
    TORCH_CHECK(Y_lm.size(0) == N, "Y_lm must have N rows");
    TORCH_CHECK(Y_lm.size(1) == K, "Y_lm must have (L_max+1)^2 columns");
    TORCH_CHECK(Y_lm.dtype() == torch::kFloat32, "Y_lm must be float32");
    if (N == 0) return;
    const c10::DeviceGuard guard(edge_vectors.device());
    check_status(batteries_spherical_harmonics(cptr<float>(edge_vectors, "edge_vectors"),
                                               mptr<float>(Y_lm, "Y_lm"), N, (int)L_max, 0,
                                               current_stream(edge_vectors)),
                 "spherical_harmonics_inplace");
}

torch::Tensor sh_backward_impl(const torch::Tensor& v, const torch::Tensor& g, int normalize) {
    check_vectors(v);
    TORCH_CHECK(g.dim() == 2, "grad_Y_lm must be 2D");
    TORCH_CHECK(v.size(0) == g.size(0), "Batch sizes must match");
    TORCH_CHECK(g.dtype() == torch::kFloat32, "grad_Y_lm must be float32");
    int L_max = -1;
    for (int l = 0; l <= 6; ++l)
        if ((l + 1) * (l + 1) == g.size(1)) L_max = l;
    TORCH_CHECK(L_max >= 0, "Invalid number of components: ", g.size(1));
    const int64_t N = v.size(0);
    torch::Tensor out = torch::empty({N, 3}, f32_like(v));
    if (N == 0) return out;
    const c10::DeviceGuard guard(v.device());
    check_status(batteries_spherical_harmonics_backward(
                     cptr<float>(v, "edge_vectors"), cptr<float>(g, "grad_Y_lm"),
                     mptr<float>(out, "grad_xyz"), N, L_max, normalize, current_stream(v)),
                 "spherical_harmonics_backward");
    return out;
}

torch::Tensor spherical_harmonics_backward(const torch::Tensor& edge_vectors,
                                           const torch::Tensor& grad_Y_lm) {
    return sh_backward_impl(edge_vectors, grad_Y_lm, 0);
}

// Extension: gradient w.r.t. the raw vector of spherical_harmonics_normalized.
torch::Tensor spherical_harmonics_normalized_backward(const torch::Tensor& edge_vectors,
                                                      const torch::Tensor& grad_Y_lm) {
    return sh_backward_impl(edge_vectors, grad_Y_lm, 1);
}

// ---------------------------------------------------------------------------
// tensor products (reference bindings.cpp:120-227, 285-393)
// ---------------------------------------------------------------------------
torch::Tensor tensor_product_simple(const torch::Tensor& input1, const torch::Tensor& input2) {
    TORCH_CHECK(input1.dim() == 2, "input1 must be 2D [N, 16]");
    TORCH_CHECK(input2.dim() == 2, "input2 must be 2D [N, 16]");
    TORCH_CHECK(input1.size(1) == 16, "input1 must have 16 components (L_max=3)");
    TORCH_CHECK(input2.size(1) == 16, "input2 must have 16 components (L_max=3)");
    TORCH_CHECK(input1.size(0) == input2.size(0), "input1 and input2 must have same N");
    TORCH_CHECK(input1.dtype() == torch::kFloat32, "input1 must be float32");
    TORCH_CHECK(input2.dtype() == torch::kFloat32, "input2 must be float32");
    const int64_t N = input1.size(0);
    torch::Tensor out = torch::empty({N, 16}, f32_like(input1));
    if (N == 0) return out;
    const c10::DeviceGuard guard(input1.device());
    const torch::Tensor x1 = aligned16(input1), x2 = aligned16(input2);
    check_status(batteries_tensor_product_simple_l3(cptr<float>(x1, "input1"),
                                                    cptr<float>(x2, "input2"),
                                                    mptr<float>(out, "output"), N,
                                                    current_stream(input1)),
                 "tensor_product_simple");
    return out;
}

torch::Tensor tensor_product(const torch::Tensor& input1, const torch::Tensor& input2,
                             const torch::Tensor& weights) {
    TORCH_CHECK(input1.dim() == 3, "input1 must be 3D [N, C_in, 16]");
    TORCH_CHECK(input2.dim() == 2, "input2 must be 2D [N, 16]");
    TORCH_CHECK(weights.dim() == 3, "weights must be 3D [num_paths, C_in, C_out]");
    TORCH_CHECK(input1.size(2) == 16, "input1 must have 16 components (L_max=3)");
    TORCH_CHECK(input2.size(1) == 16, "input2 must have 16 components (L_max=3)");
    TORCH_CHECK(input1.size(0) == input2.size(0), "input1 and input2 must have same N");
    TORCH_CHECK(input1.dtype() == torch::kFloat32, "input1 must be float32");
    TORCH_CHECK(input2.dtype() == torch::kFloat32, "input2 must be float32");
    TORCH_CHECK(weights.dtype() == torch::kFloat32, "weights must be float32");
    const int64_t N = input1.size(0);
    const int64_t C_in = input1.size(1);
    const int64_t C_out = weights.size(2);
    const int num_paths = batteries_get_num_paths_l3();
    TORCH_CHECK(weights.size(0) == num_paths, "weights must have ", num_paths, " paths");
    TORCH_CHECK(weights.size(1) == C_in, "weights C_in must match input1");
    TORCH_CHECK(C_in > 0 && C_out > 0, "C_in and C_out must be positive");
    torch::Tensor out = torch::empty({N, C_out, 16}, f32_like(input1));
    if (N == 0) return out;
    const c10::DeviceGuard guard(input1.device());
    check_status(batteries_tensor_product_l3(cptr<float>(input1, "input1"),
                                             cptr<float>(input2, "input2"),
                                             cptr<float>(weights, "weights"),
                                             mptr<float>(out, "output"), N, (int)C_in, (int)C_out,
                                             current_stream(input1)),
                 "tensor_product");
    return out;
}

torch::Tensor get_tp_path_info() {
    const int n = batteries_get_num_paths_l3();
    torch::Tensor info = torch::empty({n, 3}, torch::TensorOptions().dtype(torch::kInt32));
    batteries_get_path_info_l3(info.data_ptr<int>());
    return info;
}

int get_tp_num_paths() { return batteries_get_num_paths_l3(); }

std::tuple<torch::Tensor, torch::Tensor> tensor_product_simple_backward(
    const torch::Tensor& input1, const torch::Tensor& input2, const torch::Tensor& grad_output) {
    TORCH_CHECK(input1.dim() == 2 && input1.size(1) == 16, "input1 must be [N, 16]");
    TORCH_CHECK(input2.dim() == 2 && input2.size(1) == 16, "input2 must be [N, 16]");
    TORCH_CHECK(grad_output.dim() == 2 && grad_output.size(1) == 16,
                "grad_output must be [N, 16]");
    TORCH_CHECK(input1.size(0) == input2.size(0), "Batch sizes must match");
    TORCH_CHECK(input1.size(0) == grad_output.size(0), "Batch sizes must match");
    TORCH_CHECK(input1.dtype() == torch::kFloat32 && input2.dtype() == torch::kFloat32 &&
                    grad_output.dtype() == torch::kFloat32,
                "inputs must be float32");
    const int64_t N = input1.size(0);
    torch::Tensor g1 = torch::empty({N, 16}, f32_like(input1));
    torch::Tensor g2 = torch::empty({N, 16}, f32_like(input1));
    if (N == 0) return {g1, g2};
    const c10::DeviceGuard guard(input1.device());
    const torch::Tensor x1 = aligned16(input1), x2 = aligned16(input2),
                        go = aligned16(grad_output);
    check_status(batteries_tensor_product_simple_backward_l3(
                     cptr<float>(x1, "input1"), cptr<float>(x2, "input2"),
                     cptr<float>(go, "grad_output"), mptr<float>(g1, "grad_input1"),
                     mptr<float>(g2, "grad_input2"), N, current_stream(input1)),
                 "tensor_product_simple_backward");
    return {g1, g2};
}

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> tensor_product_backward(
    const torch::Tensor& input1, const torch::Tensor& input2, const torch::Tensor& weights,
    const torch::Tensor& grad_output, bool needs_input1_grad, bool needs_input2_grad,
    bool needs_weights_grad) {
    TORCH_CHECK(input1.dim() == 3, "input1 must be 3D [N, C_in, 16]");
    TORCH_CHECK(input2.dim() == 2, "input2 must be 2D [N, 16]");
    TORCH_CHECK(weights.dim() == 3, "weights must be 3D [num_paths, C_in, C_out]");
    TORCH_CHECK(grad_output.dim() == 3, "grad_output must be 3D [N, C_out, 16]");
    const int64_t N = input1.size(0);
    const int64_t C_in = input1.size(1);
    const int64_t C_out = weights.size(2);
    const int num_paths = batteries_get_num_paths_l3();
    TORCH_CHECK(weights.size(0) == num_paths, "weights must have ", num_paths, " paths");
    TORCH_CHECK(input1.size(2) == 16 && input2.size(1) == 16, "inputs must have 16 components");
    TORCH_CHECK(input2.size(0) == N && grad_output.size(0) == N, "Batch sizes must match");
    TORCH_CHECK(weights.size(1) == C_in, "weights C_in must match input1");
    TORCH_CHECK(grad_output.size(1) == C_out && grad_output.size(2) == 16,
                "grad_output must be [N, C_out, 16]");
    TORCH_CHECK(input1.dtype() == torch::kFloat32 && input2.dtype() == torch::kFloat32 &&
                    weights.dtype() == torch::kFloat32 && grad_output.dtype() == torch::kFloat32,
                "inputs must be float32");
    auto opt = f32_like(input1);
    torch::Tensor g1, g2, gW;
    if (needs_input1_grad) g1 = torch::empty({N, C_in, 16}, opt);
    if (needs_input2_grad) g2 = torch::empty({N, 16}, opt);
    if (needs_weights_grad) gW = torch::empty({num_paths, C_in, C_out}, opt);
    if (N == 0) {
        if (!g1.defined()) g1 = torch::empty({0, C_in, 16}, opt);
        if (!g2.defined()) g2 = torch::empty({0, 16}, opt);
        if (!gW.defined()) gW = torch::zeros({num_paths, C_in, C_out}, opt);
        else gW.zero_();
        return {g1, g2, gW};
    }
    const c10::DeviceGuard guard(input1.device());
    torch::Tensor ws;
    size_t wsb = 0;
    if (needs_weights_grad) {  // grad_W partials of the row segments
        wsb = batteries_tensor_product_backward_workspace_bytes(N, (int)C_in, (int)C_out);
        ws = torch::empty({(int64_t)((wsb + 3) / 4)}, opt);
    }
    check_status(batteries_tensor_product_backward_l3(
                     cptr<float>(input1, "input1"), cptr<float>(input2, "input2"),
                     cptr<float>(weights, "weights"), cptr<float>(grad_output, "grad_output"),
                     needs_input1_grad ? mptr<float>(g1, "grad_input1") : nullptr,
                     needs_input2_grad ? mptr<float>(g2, "grad_input2") : nullptr,
                     needs_weights_grad ? mptr<float>(gW, "grad_weights") : nullptr, N, (int)C_in,
                     (int)C_out, ws.defined() ? ws.data_ptr() : nullptr, wsb,
                     current_stream(input1)),
                 "tensor_product_backward");
    return {g1, g2, gW};
}

// ---------------------------------------------------------------------------
// message passing (reference bindings.cpp:402-595)
// ---------------------------------------------------------------------------
std::tuple<torch::Tensor, torch::Tensor> edge_index_to_csr(const torch::Tensor& edge_index,
                                                           int64_t N_atoms) {
    TORCH_CHECK(edge_index.dim() == 2, "edge_index must be 2D [2, N_edges]");
    TORCH_CHECK(edge_index.size(0) == 2, "edge_index first dim must be 2");
    TORCH_CHECK(edge_index.dtype() == torch::kInt64, "edge_index must be int64");
    TORCH_CHECK(N_atoms >= 0, "N_atoms must be non-negative");
    const int64_t E = edge_index.size(1);
    auto opt = torch::TensorOptions().dtype(torch::kInt64).device(edge_index.device());
    torch::Tensor row_ptr = torch::empty({N_atoms + 1}, opt);
    torch::Tensor col_idx = torch::empty({E}, opt);
    const c10::DeviceGuard guard(edge_index.device());
    const size_t wsb = batteries_edge_index_to_csr_workspace_bytes(N_atoms);
    torch::Tensor ws = torch::empty({std::max<int64_t>(1, N_atoms)}, opt);
    check_status(batteries_edge_index_to_csr(cptr<int64_t>(edge_index, "edge_index"),
                                             mptr<int64_t>(row_ptr, "row_ptr"),
                                             mptr<int64_t>(col_idx, "col_idx"), N_atoms, E,
                                             ws.data_ptr(), wsb, current_stream(edge_index)),
                 "edge_index_to_csr");
    return {row_ptr, col_idx};
}

void check_features(const torch::Tensor& x, const char* name) {
    TORCH_CHECK(x.dim() == 3, name, " must be 3D [N_atoms, C, 16]");
    TORCH_CHECK(x.size(2) == 16, name, " must have 16 irrep components");
    TORCH_CHECK(x.dtype() == torch::kFloat32, name, " must be float32");
    TORCH_CHECK(x.size(1) > 0, name, " must have at least one channel");
}

torch::Tensor fused_message_passing_simple(const torch::Tensor& node_features,
                                           const torch::Tensor& edge_vectors,
                                           const torch::Tensor& edge_index,
                                           const torch::Tensor& row_ptr,
                                           const torch::Tensor& col_idx) {
    check_features(node_features, "node_features");
    TORCH_CHECK(edge_vectors.dim() == 2, "edge_vectors must be 2D [N_edges, 3]");
    TORCH_CHECK(edge_vectors.size(1) == 3, "edge_vectors must have shape [N_edges, 3]");
    TORCH_CHECK(edge_index.dim() == 2, "edge_index must be 2D [2, N_edges]");
    TORCH_CHECK(edge_index.size(0) == 2, "edge_index first dim must be 2");
    TORCH_CHECK(edge_vectors.dtype() == torch::kFloat32, "edge_vectors must be float32");
    TORCH_CHECK(edge_index.dtype() == torch::kInt64, "edge_index must be int64");
    TORCH_CHECK(row_ptr.dtype() == torch::kInt64, "row_ptr must be int64");
    TORCH_CHECK(col_idx.dtype() == torch::kInt64, "col_idx must be int64");
    const int64_t N = node_features.size(0);
    const int64_t E = edge_vectors.size(0);
    const int64_t C = node_features.size(1);
    TORCH_CHECK(edge_index.size(1) == E, "edge_index must have N_edges columns");
    TORCH_CHECK(row_ptr.numel() == N + 1, "row_ptr must have N_atoms + 1 entries");
    TORCH_CHECK(col_idx.numel() == E, "col_idx must have N_edges entries");
    torch::Tensor out = torch::empty({N, C, 16}, f32_like(node_features));
    if (N == 0) return out;
    const c10::DeviceGuard guard(node_features.device());
    torch::Tensor x = aligned16(node_features);
    check_status(batteries_fused_message_passing_simple(
                     cptr<float>(x, "node_features"), cptr<float>(edge_vectors, "edge_vectors"),
                     cptr<int64_t>(edge_index, "edge_index"), cptr<int64_t>(row_ptr, "row_ptr"),
                     cptr<int64_t>(col_idx, "col_idx"), mptr<float>(out, "output"), N, E, (int)C,
                     current_stream(node_features)),
                 "fused_message_passing_simple");
    return out;
}

torch::Tensor fused_message_passing(const torch::Tensor& node_features,
                                    const torch::Tensor& edge_vectors,
                                    const torch::Tensor& weights, const torch::Tensor& row_ptr,
                                    const torch::Tensor& col_idx) {
    check_features(node_features, "node_features");
    TORCH_CHECK(edge_vectors.dim() == 2, "edge_vectors must be 2D [N_edges, 3]");
    TORCH_CHECK(edge_vectors.size(1) == 3, "edge_vectors must have shape [N_edges, 3]");
    TORCH_CHECK(weights.dim() == 2, "weights must be 2D [C_in, C_out]");
    TORCH_CHECK(edge_vectors.dtype() == torch::kFloat32, "edge_vectors must be float32");
    TORCH_CHECK(weights.dtype() == torch::kFloat32, "weights must be float32");
    TORCH_CHECK(row_ptr.dtype() == torch::kInt64, "row_ptr must be int64");
    TORCH_CHECK(col_idx.dtype() == torch::kInt64, "col_idx must be int64");
    const int64_t N = node_features.size(0);
    const int64_t E = edge_vectors.size(0);
    const int64_t C_in = node_features.size(1);
    const int64_t C_out = weights.size(1);
    TORCH_CHECK(weights.size(0) == C_in, "weights first dim must match C_in");
    TORCH_CHECK(row_ptr.numel() == N + 1, "row_ptr must have N_atoms + 1 entries");
    TORCH_CHECK(col_idx.numel() == E, "col_idx must have N_edges entries");
    torch::Tensor out = torch::empty({N, C_out, 16}, f32_like(node_features));
    if (N == 0) return out;
    const c10::DeviceGuard guard(node_features.device());
    torch::Tensor x = aligned16(node_features);
    const size_t wsb = batteries_fused_message_passing_workspace_bytes(N, (int)C_in);
    torch::Tensor ws = torch::empty({N, C_in, 16}, f32_like(node_features));
    check_status(batteries_fused_message_passing(
                     cptr<float>(x, "node_features"), cptr<float>(edge_vectors, "edge_vectors"),
                     cptr<float>(weights, "weights"), cptr<int64_t>(row_ptr, "row_ptr"),
                     cptr<int64_t>(col_idx, "col_idx"), mptr<float>(out, "output"), N, E,
                     (int)C_in, (int)C_out, ws.data_ptr(), wsb, current_stream(node_features)),
                 "fused_message_passing");
    return out;
}

torch::Tensor fused_sh_tp_simple(const torch::Tensor& edge_vectors,
                                 const torch::Tensor& node_features,
                                 const torch::Tensor& source_idx) {
    TORCH_CHECK(edge_vectors.dim() == 2, "edge_vectors must be 2D [N_edges, 3]");
    TORCH_CHECK(edge_vectors.size(1) == 3, "edge_vectors must have shape [N_edges, 3]");
    check_features(node_features, "node_features");
    TORCH_CHECK(source_idx.dim() == 1, "source_idx must be 1D [N_edges]");
    TORCH_CHECK(edge_vectors.dtype() == torch::kFloat32, "edge_vectors must be float32");
    TORCH_CHECK(source_idx.dtype() == torch::kInt64, "source_idx must be int64");
    const int64_t E = edge_vectors.size(0);
    const int64_t C = node_features.size(1);
    TORCH_CHECK(source_idx.size(0) == E, "source_idx must have N_edges elements");
    torch::Tensor msg = torch::empty({E, C, 16}, f32_like(node_features));
    if (E == 0) return msg;
    const c10::DeviceGuard guard(node_features.device());
    torch::Tensor x = aligned16(node_features);
    check_status(batteries_fused_sh_tp_simple(cptr<float>(edge_vectors, "edge_vectors"),
                                              cptr<float>(x, "node_features"),
                                              cptr<int64_t>(source_idx, "source_idx"),
                                              mptr<float>(msg, "messages"), node_features.size(0),
                                              E, (int)C, 0,
                                              current_stream(node_features)),
                 "fused_sh_tp_simple");
    return msg;
}

// Extension: out[d] = sum_{k in CSR row d} TP_simple(X[source_idx[e_k]], Y(v_{e_k})),
// e_k = perm[k] if perm is given else k; normalize=True evaluates Y at v/|v|.
// One kernel, no messages tensor, no atomics.
torch::Tensor sh_tp_scatter(const torch::Tensor& edge_vectors, const torch::Tensor& node_features,
                            const torch::Tensor& source_idx, const torch::Tensor& row_ptr,
                            const c10::optional<torch::Tensor>& perm, bool normalize) {
    check_vectors(edge_vectors);
    check_features(node_features, "node_features");
    TORCH_CHECK(source_idx.dim() == 1 && source_idx.dtype() == torch::kInt64,
                "source_idx must be int64 [N_edges]");
    TORCH_CHECK(row_ptr.dim() == 1 && row_ptr.dtype() == torch::kInt64 && row_ptr.numel() >= 1,
                "row_ptr must be int64 [N_dst + 1]");
    const int64_t E = edge_vectors.size(0);
    const int64_t N_dst = row_ptr.numel() - 1;
    const int64_t C = node_features.size(1);
    TORCH_CHECK(source_idx.numel() == E, "source_idx must have N_edges elements");
    const int64_t* pp = nullptr;
    if (perm.has_value() && perm->defined()) {
        TORCH_CHECK(perm->dtype() == torch::kInt64 && perm->numel() == E,
                    "perm must be int64 [N_edges]");
        pp = cptr<int64_t>(*perm, "perm");
    }
    torch::Tensor out = torch::empty({N_dst, C, 16}, f32_like(node_features));
    if (N_dst == 0) return out;
    const c10::DeviceGuard guard(node_features.device());
    torch::Tensor x = aligned16(node_features);
    check_status(batteries_sh_tp_scatter_csr(cptr<float>(edge_vectors, "edge_vectors"),
                                             cptr<float>(x, "node_features"),
                                             cptr<int64_t>(source_idx, "source_idx"), pp,
                                             cptr<int64_t>(row_ptr, "row_ptr"),
                                             mptr<float>(out, "output"), node_features.size(0),
                                             N_dst, E, (int)C, normalize ? 1 : 0,
                                             current_stream(node_features)),
                 "sh_tp_scatter");
    return out;
}

// Extension: the weighted scatter, out[d] = sum_{k in CSR row d}
// tensor_product(X[source_idx[e_k]], Y(v_{e_k}), weights) with e_k = perm[k] if perm
// is given else k -- the reference's interaction block SH -> tensor_product ->
// scatter_add (benchmarks/benchmark_e2e_mace.py:308-349) without the per-edge
// messages.  order (optional) lists the destinations in the order they are
// processed (any permutation of 0..N_dst-1; a spatial order keeps source rows in L2).
torch::Tensor sh_tp_scatter_weighted(const torch::Tensor& edge_vectors,
                                     const torch::Tensor& node_features,
                                     const torch::Tensor& weights, const torch::Tensor& source_idx,
                                     const torch::Tensor& row_ptr,
                                     const c10::optional<torch::Tensor>& perm,
                                     const c10::optional<torch::Tensor>& order, bool normalize) {
    check_vectors(edge_vectors);
    check_features(node_features, "node_features");
    TORCH_CHECK(weights.dim() == 3, "weights must be 3D [num_paths, C_in, C_out]");
    TORCH_CHECK(weights.dtype() == torch::kFloat32, "weights must be float32");
    check_device(weights, "weights");
    const int num_paths = batteries_get_num_paths_l3();
    TORCH_CHECK(weights.size(0) == num_paths, "weights must have ", num_paths, " paths");
    const int64_t C_in = node_features.size(1);
    TORCH_CHECK(weights.size(1) == C_in, "weights second dim must match C_in");
    const int64_t C_out = weights.size(2);
    TORCH_CHECK(C_out > 0, "C_out must be positive");
    TORCH_CHECK(source_idx.dim() == 1 && source_idx.dtype() == torch::kInt64,
                "source_idx must be int64 [N_edges]");
    TORCH_CHECK(row_ptr.dim() == 1 && row_ptr.dtype() == torch::kInt64 && row_ptr.numel() >= 1,
                "row_ptr must be int64 [N_dst + 1]");
    const int64_t E = edge_vectors.size(0);
    const int64_t N_dst = row_ptr.numel() - 1;
    TORCH_CHECK(source_idx.numel() == E, "source_idx must have N_edges elements");
    const int64_t* pp = nullptr;
    if (perm.has_value() && perm->defined()) {
        TORCH_CHECK(perm->dtype() == torch::kInt64 && perm->numel() == E,
                    "perm must be int64 [N_edges]");
        pp = cptr<int64_t>(*perm, "perm");
    }
    const int64_t* op = nullptr;
    if (order.has_value() && order->defined()) {
        TORCH_CHECK(order->dtype() == torch::kInt64 && order->numel() == N_dst,
                    "order must be int64 [N_dst]");
        op = cptr<int64_t>(*order, "order");
    }
    torch::Tensor out = torch::empty({N_dst, C_out, 16}, f32_like(node_features));
    if (N_dst == 0) return out;
    TORCH_CHECK(E == 0 || node_features.size(0) > 0, "edges need source nodes");
    const c10::DeviceGuard guard(node_features.device());
    torch::Tensor x = aligned16(node_features);
    torch::Tensor w = weights.contiguous();
    const size_t wsb =
        batteries_sh_tp_scatter_weighted_workspace_bytes(N_dst, E, (int)C_in, (int)C_out);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 15) / 16), 4}, f32_like(node_features));
    check_status(batteries_sh_tp_scatter_weighted(
                     cptr<float>(edge_vectors, "edge_vectors"), cptr<float>(x, "node_features"),
                     cptr<float>(w, "weights"), cptr<int64_t>(source_idx, "source_idx"), pp,
                     cptr<int64_t>(row_ptr, "row_ptr"), op, mptr<float>(out, "output"),
                     node_features.size(0), N_dst, E, (int)C_in, (int)C_out, normalize ? 1 : 0,
                     ws.data_ptr(), wsb, current_stream(node_features)),
                 "sh_tp_scatter_weighted");
    return out;
}

// Extension: the weighted scatter's processing order, destinations grouped by edge count
// within 16-position windows and each XCD's tiles sorted by decreasing edge count
// (batteries_weighted_tile_order).
torch::Tensor weighted_tile_order(const c10::optional<torch::Tensor>& order,
                                  const torch::Tensor& row_ptr) {
    TORCH_CHECK(row_ptr.dim() == 1 && row_ptr.dtype() == torch::kInt64 && row_ptr.numel() >= 1,
                "row_ptr must be int64 [N_dst + 1]");
    check_device(row_ptr, "row_ptr");
    const int64_t N_dst = row_ptr.numel() - 1;
    const int64_t* op = nullptr;
    if (order.has_value() && order->defined()) {
        TORCH_CHECK(order->dtype() == torch::kInt64 && order->numel() == N_dst,
                    "order must be int64 [N_dst]");
        op = cptr<int64_t>(*order, "order");
    }
    const c10::DeviceGuard guard(row_ptr.device());
    torch::Tensor out = torch::empty({N_dst}, row_ptr.options());
    check_status(batteries_weighted_tile_order(op, cptr<int64_t>(row_ptr, "row_ptr"), N_dst,
                                               mptr<int64_t>(out, "order_out"),
                                               current_stream(row_ptr)),
                 "weighted_tile_order");
    return out;
}

// Extension: atoms in Morton order of a 32^3 grid over the (orthorhombic) box.
torch::Tensor spatial_order(const torch::Tensor& positions, const torch::Tensor& cell) {
    TORCH_CHECK(positions.dim() == 2 && positions.size(1) == 3, "positions must be [N, 3]");
    TORCH_CHECK(positions.dtype() == torch::kFloat32, "positions must be float32");
    TORCH_CHECK(cell.numel() == 9, "cell must be [3, 3]");
    check_device(positions, "positions");
    const int64_t N = positions.size(0);
    torch::Tensor cell_cpu = cell.detach().to(torch::kCPU, torch::kFloat32).contiguous();
    const float* h = cell_cpu.data_ptr<float>();
    const float box[3] = {h[0], h[4], h[8]};
    auto i64 = torch::TensorOptions().dtype(torch::kInt64).device(positions.device());
    torch::Tensor order = torch::empty({N}, i64);
    if (N == 0) return order;
    const c10::DeviceGuard guard(positions.device());
    const size_t wsb = batteries_spatial_order_workspace_bytes(N);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 7) / 8)}, i64);
    check_status(batteries_spatial_order(cptr<float>(positions, "positions"), box, N,
                                         ws.data_ptr(), wsb, order.data_ptr<int64_t>(),
                                         current_stream(positions)),
                 "spatial_order");
    return order;
}

// Extension: processing schedule of the fused scatter for a CSR graph
// (row_ptr over destinations, optional col_perm as in fused_message_passing_simple)
// and a destination order.  Returns (row_ptr_s, edge_perm, row_dst, n_blocks,
// rows_per_block) for sh_tp_scatter_scheduled.
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor, int64_t, int64_t> mp_schedule(
    const torch::Tensor& row_ptr, const torch::Tensor& order, int64_t C,
    const c10::optional<torch::Tensor>& col_perm, int64_t num_edges) {
    TORCH_CHECK(row_ptr.dim() == 1 && row_ptr.dtype() == torch::kInt64 && row_ptr.numel() >= 1,
                "row_ptr must be int64 [N_dst + 1]");
    const int64_t N = row_ptr.numel() - 1;
    TORCH_CHECK(order.dim() == 1 && order.dtype() == torch::kInt64 && order.numel() == N,
                "order must be int64 [N_dst]");
    TORCH_CHECK(C > 0, "C must be positive");
    check_device(row_ptr, "row_ptr");
    check_device(order, "order");
    int nb = 0, rpb = 0;
    check_status(batteries_mp_schedule_shape(N, (int)C, &nb, &rpb), "mp_schedule");
    // E from the caller when it knows it (no host sync), else from row_ptr[N]
    const int64_t E = num_edges >= 0 ? num_edges : row_ptr[N].item<int64_t>();
    const int64_t* cp = nullptr;
    if (col_perm.has_value() && col_perm->defined()) {
        TORCH_CHECK(col_perm->dtype() == torch::kInt64 && col_perm->numel() == E,
                    "col_perm must be int64 [N_edges]");
        cp = cptr<int64_t>(*col_perm, "col_perm");
    }
    auto i64 = torch::TensorOptions().dtype(torch::kInt64).device(row_ptr.device());
    const int64_t ns = (int64_t)nb * rpb;
    torch::Tensor rps = torch::empty({ns + 1}, i64);
    torch::Tensor dst = torch::empty({ns}, i64);
    torch::Tensor ep = torch::empty({E}, i64);
    const c10::DeviceGuard guard(row_ptr.device());
    const size_t wsb = batteries_mp_schedule_workspace_bytes(nb, rpb);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 7) / 8)}, i64);
    check_status(batteries_mp_schedule(cptr<int64_t>(row_ptr, "row_ptr"), cp,
                                       cptr<int64_t>(order, "order"), N, E, (int)C, nb, rpb,
                                       rps.data_ptr<int64_t>(), dst.data_ptr<int64_t>(),
                                       ep.data_ptr<int64_t>(), ws.data_ptr(), wsb,
                                       current_stream(row_ptr)),
                 "mp_schedule");
    return {rps, ep, dst, (int64_t)nb, (int64_t)rpb};
}

// Extension: sh_tp_scatter driven by an mp_schedule (same result, spatial order).
torch::Tensor sh_tp_scatter_scheduled(const torch::Tensor& edge_vectors,
                                      const torch::Tensor& node_features,
                                      const torch::Tensor& source_idx,
                                      const torch::Tensor& row_ptr_s,
                                      const torch::Tensor& edge_perm, const torch::Tensor& row_dst,
                                      int64_t n_blocks, int64_t rows_per_block, int64_t N_dst,
                                      bool normalize, bool channel_split) {
    check_vectors(edge_vectors);
    check_features(node_features, "node_features");
    const int64_t E = edge_vectors.size(0);
    const int64_t C = node_features.size(1);
    TORCH_CHECK(source_idx.dtype() == torch::kInt64 && source_idx.numel() == E,
                "source_idx must be int64 [N_edges]");
    TORCH_CHECK(edge_perm.dtype() == torch::kInt64 && edge_perm.numel() == E,
                "edge_perm must be int64 [N_edges]");
    TORCH_CHECK(n_blocks > 0 && n_blocks % 8 == 0 && rows_per_block > 0, "invalid schedule shape");
    const int64_t ns = n_blocks * rows_per_block;
    TORCH_CHECK(row_ptr_s.dtype() == torch::kInt64 && row_ptr_s.numel() == ns + 1,
                "row_ptr_s must be int64 [n_blocks * rows_per_block + 1]");
    TORCH_CHECK(row_dst.dtype() == torch::kInt64 && row_dst.numel() == ns,
                "row_dst must be int64 [n_blocks * rows_per_block]");
    TORCH_CHECK(N_dst >= 0 && N_dst <= ns, "N_dst out of range");
    torch::Tensor out = torch::empty({N_dst, C, 16}, f32_like(node_features));
    if (N_dst == 0) return out;
    const c10::DeviceGuard guard(node_features.device());
    torch::Tensor x = aligned16(node_features);
    auto run = channel_split ? batteries_sh_tp_scatter_scheduled_chsplit
                             : batteries_sh_tp_scatter_scheduled;
    check_status(run(cptr<float>(edge_vectors, "edge_vectors"), cptr<float>(x, "node_features"),
                     cptr<int64_t>(source_idx, "source_idx"), cptr<int64_t>(row_ptr_s, "row_ptr_s"),
                     cptr<int64_t>(edge_perm, "edge_perm"), cptr<int64_t>(row_dst, "row_dst"),
                     (int)n_blocks, (int)rows_per_block, mptr<float>(out, "output"),
                     node_features.size(0), E, (int)C, normalize ? 1 : 0,
                     current_stream(node_features)),
                 "sh_tp_scatter_scheduled");
    return out;
}

// Extension (torch-level form of the reference's ctypes neighbor list):
// returns (edge_index int64 [2, E] with row 0 = i, row 1 = j sorted by (i, j),
// edge_vectors [E, 3] = minimum-image pos[j] - pos[i], row_offsets int64 [N+1]).
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> neighbor_list(
    const torch::Tensor& positions, const torch::Tensor& cell, double cutoff, bool self_loops,
    int64_t row_capacity) {
    TORCH_CHECK(positions.dim() == 2 && positions.size(1) == 3, "positions must be [N, 3]");
    TORCH_CHECK(positions.dtype() == torch::kFloat32, "positions must be float32");
    TORCH_CHECK(cell.numel() == 9, "cell must be [3, 3]");
    check_device(positions, "positions");
    const int64_t N = positions.size(0);
    torch::Tensor cell_cpu = cell.detach().to(torch::kCPU, torch::kFloat32).contiguous();
    const float* h = cell_cpu.data_ptr<float>();
    const float box[3] = {h[0], h[4], h[8]};
    const float rc = (float)cutoff;
    TORCH_CHECK(row_capacity <= 1 << 20, "row_capacity out of range");
    auto i64 = torch::TensorOptions().dtype(torch::kInt64).device(positions.device());
    auto i32 = torch::TensorOptions().dtype(torch::kInt32).device(positions.device());
    const c10::DeviceGuard guard(positions.device());
    hipStream_t s = current_stream(positions);
    // up to 8192 atoms: three kernels and a scan (row_capacity < 0 takes the passes below)
    const size_t cwsb = row_capacity >= 0
                            ? batteries_neighbor_list_cells_workspace_bytes(N, box, rc, (int)row_capacity)
                            : 0;
    if (cwsb > 0) {
        torch::Tensor ws = torch::empty({(int64_t)((cwsb + 7) / 8)}, i64);
        torch::Tensor offsets = torch::empty({N + 2}, i64);  // [N+1] and E once more
        check_status(batteries_neighbor_list_cells_count(
                         cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0,
                         (int)row_capacity, ws.data_ptr(), cwsb, offsets.data_ptr<int64_t>(),
                         nullptr, s),
                     "neighbor_list");
        const int64_t E = offsets[N].item<int64_t>();  // one host sync, as in the reference
        torch::Tensor edge_index = torch::empty({2, E}, i64);
        torch::Tensor vec = torch::empty({E, 3}, f32_like(positions));
        check_status(batteries_neighbor_list_cells_write_i64(
                         cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0,
                         (int)row_capacity, ws.data_ptr(), cwsb, offsets.data_ptr<int64_t>(), E,
                         E ? edge_index.data_ptr<int64_t>() : nullptr,
                         E ? vec.data_ptr<float>() : nullptr, s),
                     "neighbor_list");
        return {edge_index, vec, offsets.narrow(0, 0, N + 1)};
    }
    const size_t wsb = batteries_neighbor_list_workspace_bytes(N, box, rc);
    TORCH_CHECK(wsb > 0, "invalid cell or cutoff");
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 7) / 8)}, i64);
    torch::Tensor total = torch::empty({1}, i64);
    check_status(batteries_neighbor_list_count(cptr<float>(positions, "positions"), box, N, rc,
                                               self_loops ? 1 : 0, ws.data_ptr(), wsb,
                                               total.data_ptr<int64_t>(), s),
                 "neighbor_list");
    const int64_t E = total.item<int64_t>();  // one host sync, as in the reference
    torch::Tensor tmp_j = torch::empty({E}, i32);
    torch::Tensor tmp_vec = torch::empty({E, 3}, f32_like(positions));
    torch::Tensor edge_index = torch::empty({2, E}, i64);
    torch::Tensor vec = torch::empty({E, 3}, f32_like(positions));
    check_status(batteries_neighbor_list_write_i64(
                     cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0,
                     ws.data_ptr(), wsb, E, tmp_j.data_ptr<int>(), tmp_vec.data_ptr<float>(),
                     edge_index.data_ptr<int64_t>(), vec.data_ptr<float>(), nullptr, s),
                 "neighbor_list");
    // the row offsets copied out of the workspace, so the result owns its own [N+1]
    // tensor (neighbor_graph, below, keeps the zero-copy view for batmobile.Graph)
    const size_t at = batteries_neighbor_list_offsets_at(N, box, rc);
    TORCH_CHECK(at > 0 && at % 8 == 0, "neighbor_list: workspace layout");
    torch::Tensor offsets = ws.narrow(0, (int64_t)(at / 8), N + 1).clone();
    return {edge_index, vec, offsets};
}

// Extension for batmobile.Graph: the neighbor list in the message-passing layout,
// (src int64 [E] = j, dst int64 [E] = i, edge_vectors [E, 3] = minimum-image
// pos[i] - pos[j], row_offsets int64 [N+1], spatial order int64 [N]), edges
// grouped by destination i and src ascending within; the neighbor_list result read
// with roles swapped.
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor> neighbor_graph(
    const torch::Tensor& positions, const torch::Tensor& cell, double cutoff, bool self_loops) {
    TORCH_CHECK(positions.dim() == 2 && positions.size(1) == 3, "positions must be [N, 3]");
    TORCH_CHECK(positions.dtype() == torch::kFloat32, "positions must be float32");
    TORCH_CHECK(cell.numel() == 9, "cell must be [3, 3]");
    check_device(positions, "positions");
    const int64_t N = positions.size(0);
    torch::Tensor cell_cpu = cell.detach().to(torch::kCPU, torch::kFloat32).contiguous();
    const float* h = cell_cpu.data_ptr<float>();
    const float box[3] = {h[0], h[4], h[8]};
    const float rc = (float)cutoff;
    const size_t wsb = batteries_neighbor_list_workspace_bytes(N, box, rc);
    TORCH_CHECK(wsb > 0, "invalid cell or cutoff");
    auto i64 = torch::TensorOptions().dtype(torch::kInt64).device(positions.device());
    auto i32 = torch::TensorOptions().dtype(torch::kInt32).device(positions.device());
    const c10::DeviceGuard guard(positions.device());
    hipStream_t s = current_stream(positions);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 7) / 8)}, i64);
    torch::Tensor total = torch::empty({1}, i64);
    check_status(batteries_neighbor_list_count(cptr<float>(positions, "positions"), box, N, rc,
                                               self_loops ? 1 : 0, ws.data_ptr(), wsb,
                                               total.data_ptr<int64_t>(), s),
                 "neighbor_graph");
    const int64_t E = total.item<int64_t>();  // one host sync, as in the reference
    torch::Tensor tmp_j = torch::empty({E}, i32);
    torch::Tensor tmp_vec = torch::empty({E, 3}, f32_like(positions));
    torch::Tensor src = torch::empty({E}, i64);
    torch::Tensor dst = torch::empty({E}, i64);
    torch::Tensor vec = torch::empty({E, 3}, f32_like(positions));
    torch::Tensor order = torch::empty({N}, i64);
    check_status(batteries_neighbor_graph_write(
                     cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0,
                     ws.data_ptr(), wsb, tmp_j.data_ptr<int>(), tmp_vec.data_ptr<float>(),
                     src.data_ptr<int64_t>(), dst.data_ptr<int64_t>(), vec.data_ptr<float>(),
                     nullptr, order.data_ptr<int64_t>(), s),
                 "neighbor_graph");
    // the row offsets read in place from the workspace (a view that keeps it alive)
    const size_t at = batteries_neighbor_list_offsets_at(N, box, rc);
    TORCH_CHECK(at > 0 && at % 8 == 0, "neighbor_graph: workspace layout");
    torch::Tensor offsets = ws.narrow(0, (int64_t)(at / 8), N + 1);
    return {src, dst, vec, offsets, order};
}

// The same with arrays of `capacity` edges and no host synchronisation: the edge
// count stays on the device (offsets[N]); overflow [1] int32 is 1 when it exceeded
// the capacity (then every row is empty).
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor, torch::Tensor>
neighbor_graph_capacity(const torch::Tensor& positions, const torch::Tensor& cell, double cutoff,
                        bool self_loops, int64_t capacity) {
    TORCH_CHECK(positions.dim() == 2 && positions.size(1) == 3, "positions must be [N, 3]");
    TORCH_CHECK(positions.dtype() == torch::kFloat32, "positions must be float32");
    TORCH_CHECK(cell.numel() == 9, "cell must be [3, 3]");
    TORCH_CHECK(capacity >= 0, "capacity must be >= 0");
    check_device(positions, "positions");
    const int64_t N = positions.size(0);
    torch::Tensor cell_cpu = cell.detach().to(torch::kCPU, torch::kFloat32).contiguous();
    const float* h = cell_cpu.data_ptr<float>();
    const float box[3] = {h[0], h[4], h[8]};
    const float rc = (float)cutoff;
    const size_t wsb = batteries_neighbor_list_workspace_bytes(N, box, rc);
    TORCH_CHECK(wsb > 0, "invalid cell or cutoff");
    auto i64 = torch::TensorOptions().dtype(torch::kInt64).device(positions.device());
    auto i32 = torch::TensorOptions().dtype(torch::kInt32).device(positions.device());
    const c10::DeviceGuard guard(positions.device());
    hipStream_t s = current_stream(positions);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 7) / 8)}, i64);
    check_status(batteries_neighbor_list_count(cptr<float>(positions, "positions"), box, N, rc,
                                               self_loops ? 1 : 0, ws.data_ptr(), wsb, nullptr, s),
                 "neighbor_graph_capacity");
    torch::Tensor tmp_j = torch::empty({capacity}, i32);
    torch::Tensor tmp_vec = torch::empty({capacity, 3}, f32_like(positions));
    torch::Tensor src = torch::empty({capacity}, i64);
    torch::Tensor dst = torch::empty({capacity}, i64);
    torch::Tensor vec = torch::empty({capacity, 3}, f32_like(positions));
    torch::Tensor order = torch::empty({N}, i64);
    torch::Tensor overflow = torch::empty({1}, i32);
    check_status(batteries_neighbor_graph_write_capacity(
                     cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0,
                     ws.data_ptr(), wsb, capacity, capacity ? tmp_j.data_ptr<int>() : nullptr,
                     capacity ? tmp_vec.data_ptr<float>() : nullptr,
                     capacity ? src.data_ptr<int64_t>() : nullptr,
                     capacity ? dst.data_ptr<int64_t>() : nullptr,
                     capacity ? vec.data_ptr<float>() : nullptr, nullptr,
                     order.data_ptr<int64_t>(), overflow.data_ptr<int>(), s),
                 "neighbor_graph_capacity");
    const size_t at = batteries_neighbor_list_offsets_at(N, box, rc);
    TORCH_CHECK(at > 0 && at % 8 == 0, "neighbor_graph_capacity: workspace layout");
    torch::Tensor offsets = ws.narrow(0, (int64_t)(at / 8), N + 1);
    return {src, dst, vec, offsets, order, overflow};
}

// Extension for batmobile.Graph: the whole build (neighbor list in the message-passing
// layout, spatial order, schedule) by batteries_graph_build_count / _write, for the
// systems within its limits; None otherwise (the caller then uses neighbor_graph and
// mp_schedule, which give the same results).  max_edges < 0: arrays of exactly E edges
// (one host synchronisation for E); else arrays of max_edges edges, no host
// synchronisation, overflow [1] int32 as in neighbor_graph_capacity.
// Returns (src, dst, edge_vectors, row_offsets, order, row_ptr_s, edge_perm, row_dst,
// n_blocks, rows_per_block, overflow or None).
pybind11::object graph_build(const torch::Tensor& positions, const torch::Tensor& cell,
                             double cutoff, bool self_loops, int64_t C, int64_t max_edges,
                             int64_t row_capacity) {
    TORCH_CHECK(positions.dim() == 2 && positions.size(1) == 3, "positions must be [N, 3]");
    TORCH_CHECK(positions.dtype() == torch::kFloat32, "positions must be float32");
    TORCH_CHECK(cell.numel() == 9, "cell must be [3, 3]");
    TORCH_CHECK(C > 0 && C <= INT32_MAX, "C must be positive");
    TORCH_CHECK(row_capacity >= 0 && row_capacity <= 1 << 20, "row_capacity out of range");
    check_device(positions, "positions");
    const int64_t N = positions.size(0);
    torch::Tensor cell_cpu = cell.detach().to(torch::kCPU, torch::kFloat32).contiguous();
    const float* h = cell_cpu.data_ptr<float>();
    const float box[3] = {h[0], h[4], h[8]};
    const float rc = (float)cutoff;
    const size_t wsb = batteries_graph_build_workspace_bytes(N, box, rc, (int)C, (int)row_capacity);
    if (wsb == 0) return pybind11::none();
    int nb = 0, rpb = 0;
    check_status(batteries_mp_schedule_shape(N, (int)C, &nb, &rpb), "graph_build");
    const int64_t ns = (int64_t)nb * rpb;
    auto i64 = torch::TensorOptions().dtype(torch::kInt64).device(positions.device());
    auto i32 = torch::TensorOptions().dtype(torch::kInt32).device(positions.device());
    const c10::DeviceGuard guard(positions.device());
    hipStream_t s = current_stream(positions);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 7) / 8)}, i64);
    // the per-atom and per-slot results in one allocation
    torch::Tensor meta = torch::empty({(N + 1) + N + (ns + 1) + ns}, i64);
    torch::Tensor row_ptr = meta.narrow(0, 0, N + 1);
    torch::Tensor order = meta.narrow(0, N + 1, N);
    torch::Tensor rps = meta.narrow(0, 2 * N + 1, ns + 1);
    torch::Tensor rdst = meta.narrow(0, 2 * N + 2 + ns, ns);
    torch::Tensor overflow = torch::empty({1}, i32);
    check_status(batteries_graph_build_count(
                     cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0, (int)C,
                     nb, rpb, max_edges, (int)row_capacity, ws.data_ptr(), wsb,
                     row_ptr.data_ptr<int64_t>(), order.data_ptr<int64_t>(),
                     rps.data_ptr<int64_t>(), rdst.data_ptr<int64_t>(), overflow.data_ptr<int>(),
                     s),
                 "graph_build");
    const int64_t E = max_edges < 0 ? row_ptr[N].item<int64_t>() : max_edges;  // exact: one sync
    torch::Tensor eidx = torch::empty({3 * E}, i64);  // src | dst | edge_perm
    torch::Tensor src = eidx.narrow(0, 0, E);
    torch::Tensor dst = eidx.narrow(0, E, E);
    torch::Tensor ep = eidx.narrow(0, 2 * E, E);
    torch::Tensor vec = torch::empty({E, 3}, f32_like(positions));
    if (E > 0)
        check_status(batteries_graph_build_write(
                         cptr<float>(positions, "positions"), box, N, rc, self_loops ? 1 : 0,
                         (int)row_capacity, ws.data_ptr(), wsb, row_ptr.data_ptr<int64_t>(),
                         overflow.data_ptr<int>(), src.data_ptr<int64_t>(),
                         dst.data_ptr<int64_t>(), vec.data_ptr<float>(),
                         ep.data_ptr<int64_t>(), s),
                     "graph_build");
    pybind11::object ov = max_edges < 0 ? pybind11::none() : pybind11::cast(overflow);
    return pybind11::make_tuple(src, dst, vec, row_ptr, order, rps, ep, rdst, (int64_t)nb,
                                (int64_t)rpb, ov);
}

torch::Tensor selftest_mfma_16x16x4(const torch::Tensor& A, const torch::Tensor& B) {
    TORCH_CHECK(A.numel() == 64 && B.numel() == 64 && A.dtype() == torch::kFloat32 &&
                    B.dtype() == torch::kFloat32,
                "A [16,4] and B [4,16] float32");
    torch::Tensor D = torch::empty({16, 16}, f32_like(A));
    const c10::DeviceGuard guard(A.device());
    check_status(batteries_selftest_mfma_16x16x4(cptr<float>(A, "A"), cptr<float>(B, "B"),
                                                 mptr<float>(D, "D"), current_stream(A)),
                 "selftest_mfma_16x16x4");
    return D;
}

torch::Tensor selftest_mfma_4x4x1_bcast(const torch::Tensor& A, const torch::Tensor& B) {
    TORCH_CHECK(A.numel() == 64 && B.numel() == 64 && A.dtype() == torch::kFloat32 &&
                    B.dtype() == torch::kFloat32,
                "A [64] and B [64] float32");
    torch::Tensor D = torch::empty({16, 64, 4}, f32_like(A));
    const c10::DeviceGuard guard(A.device());
    check_status(batteries_selftest_mfma_4x4x1_bcast(cptr<float>(A, "A"), cptr<float>(B, "B"),
                                                     mptr<float>(D, "D"), current_stream(A)),
                 "selftest_mfma_4x4x1_bcast");
    return D;
}

// ---------------------------------------------------------------------------
// MACE-style interaction layer with per-edge radial weights (no single
// reference function: benchmarks/benchmark_e2e_mace.py:281-434 composes the
// same steps with shared weights)
// ---------------------------------------------------------------------------
torch::Tensor gemm_f32(const torch::Tensor& A, const torch::Tensor& B, bool trans_b) {
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2, "A and B must be 2D");
    TORCH_CHECK(A.dtype() == torch::kFloat32 && B.dtype() == torch::kFloat32, "float32 only");
    const int64_t M = A.size(0), K = A.size(1);
    const int64_t N = trans_b ? B.size(0) : B.size(1);
    TORCH_CHECK((trans_b ? B.size(1) : B.size(0)) == K, "inner dimensions differ");
    TORCH_CHECK(N <= INT32_MAX && K <= INT32_MAX, "N and K must fit int32");
    torch::Tensor C = torch::empty({M, N}, f32_like(A));
    if (M == 0 || N == 0) return C;
    const c10::DeviceGuard guard(A.device());
    check_status(batteries_gemm_f32(cptr<float>(A, "A"), cptr<float>(B, "B"), mptr<float>(C, "C"),
                                    M, (int)N, (int)K, trans_b ? 1 : 0, current_stream(A)),
                 "gemm_f32");
    return C;
}

torch::Tensor mace_reverse_edges(const torch::Tensor& row_ptr, const torch::Tensor& src) {
    TORCH_CHECK(row_ptr.dtype() == torch::kInt64 && src.dtype() == torch::kInt64, "int64 indices");
    const int64_t N = row_ptr.numel() - 1, E = src.numel();
    TORCH_CHECK(N >= 0, "row_ptr must have N + 1 entries");
    torch::Tensor rev = torch::empty({E}, row_ptr.options());
    torch::Tensor missing = torch::empty({1}, row_ptr.options().dtype(torch::kInt32));
    const c10::DeviceGuard guard(row_ptr.device());
    check_status(batteries_mace_reverse_edges(cptr<int64_t>(row_ptr, "row_ptr"),
                                              cptr<int64_t>(src, "src"), mptr<int64_t>(rev, "rev"),
                                              mptr<int>(missing, "missing"), N, E,
                                              current_stream(row_ptr)),
                 "mace_reverse_edges");
    TORCH_CHECK(missing.item<int>() == 0, "mace_reverse_edges: the edge list is not symmetric");
    return rev;
}

struct MaceArgs {
    float box[3];
    int64_t N, E, C;
};

MaceArgs mace_check(const torch::Tensor& positions, const torch::Tensor& cell,
                    const torch::Tensor& x, const torch::Tensor& w1, const torch::Tensor& b1,
                    const torch::Tensor& w2, const torch::Tensor& src, const torch::Tensor& dst,
                    const torch::Tensor& row_ptr) {
    MaceArgs a;
    TORCH_CHECK(positions.dim() == 2 && positions.size(1) == 3, "positions must be [N, 3]");
    TORCH_CHECK(x.dim() == 3 && x.size(2) == 16, "node_features must be [N, C, 16]");
    a.N = positions.size(0);
    a.C = x.size(1);
    a.E = src.numel();
    TORCH_CHECK(x.size(0) == a.N, "node_features and positions disagree on N");
    TORCH_CHECK(a.C >= 1 && a.C <= 256, "C must be in [1, 256]");
    TORCH_CHECK(w1.numel() == 8 * 64 && b1.numel() == 64, "W1 [8, 64], b1 [64]");
    TORCH_CHECK(w2.dim() == 2 && w2.size(0) == 64 && w2.size(1) == 34 * a.C, "W2 must be [64, 34 C]");
    TORCH_CHECK(dst.numel() == a.E && row_ptr.numel() == a.N + 1, "edge arrays disagree");
    for (const auto* t : {&positions, &x, &w1, &b1, &w2})
        TORCH_CHECK(t->dtype() == torch::kFloat32, "float32 tensors expected");
    for (const auto* t : {&src, &dst, &row_ptr})
        TORCH_CHECK(t->dtype() == torch::kInt64, "int64 indices expected");
    TORCH_CHECK(cell.numel() == 9, "cell must be [3, 3]");
    torch::Tensor cell_cpu = cell.detach().to(torch::kCPU, torch::kFloat32).contiguous();
    const float* h = cell_cpu.data_ptr<float>();
    a.box[0] = h[0];
    a.box[1] = h[4];
    a.box[2] = h[8];
    return a;
}

// Optional processing order of the destination rows: int64 [N] on the inputs' device.
const int64_t* mace_order(const c10::optional<torch::Tensor>& order, int64_t N,
                          const torch::Tensor& like) {
    if (!order.has_value() || !order->defined()) return nullptr;
    TORCH_CHECK(order->dtype() == torch::kInt64 && order->dim() == 1 && order->numel() == N &&
                    order->device() == like.device() && order->is_contiguous(),
                "order must be a contiguous int64 [N] tensor on the device of the inputs");
    return cptr<int64_t>(*order, "order");
}

torch::Tensor mace_forward(const torch::Tensor& positions, const torch::Tensor& cell,
                           const torch::Tensor& node_features, const torch::Tensor& w1,
                           const torch::Tensor& b1, const torch::Tensor& w2,
                           const torch::Tensor& src, const torch::Tensor& dst,
                           const torch::Tensor& row_ptr, double cutoff,
                           const c10::optional<torch::Tensor>& order) {
    const MaceArgs a = mace_check(positions, cell, node_features, w1, b1, w2, src, dst, row_ptr);
    torch::Tensor x = aligned16(node_features);
    torch::Tensor out = torch::empty({a.N, a.C, 16}, f32_like(x));
    if (a.N == 0) return out;
    const int64_t* ord = mace_order(order, a.N, x);
    const c10::DeviceGuard guard(x.device());
    const size_t wsb = batteries_mace_workspace_bytes(a.N, a.E, (int)a.C, 0);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 3) / 4)}, f32_like(x));
    check_status(batteries_mace_forward(cptr<float>(positions, "positions"), a.box,
                                        cptr<float>(x, "node_features"), cptr<float>(w1, "W1"),
                                        cptr<float>(b1, "b1"), cptr<float>(w2, "W2"),
                                        cptr<int64_t>(src, "src"), cptr<int64_t>(dst, "dst"),
                                        cptr<int64_t>(row_ptr, "row_ptr"), ord,
                                        mptr<float>(out, "out"), a.N, a.E, (int)a.C,
                                        (float)cutoff, ws.data_ptr(), wsb, current_stream(x)),
                 "mace_forward");
    return out;
}

torch::Tensor mace_backward(const torch::Tensor& positions, const torch::Tensor& cell,
                            const torch::Tensor& node_features, const torch::Tensor& w1,
                            const torch::Tensor& b1, const torch::Tensor& w2,
                            const torch::Tensor& src, const torch::Tensor& dst,
                            const torch::Tensor& row_ptr, const torch::Tensor& rev,
                            const torch::Tensor& grad_out, double cutoff,
                            const c10::optional<torch::Tensor>& order) {
    const MaceArgs a = mace_check(positions, cell, node_features, w1, b1, w2, src, dst, row_ptr);
    TORCH_CHECK(rev.numel() == a.E && rev.dtype() == torch::kInt64, "rev must be int64 [E]");
    TORCH_CHECK(grad_out.dim() == 3 && grad_out.size(0) == a.N && grad_out.size(1) == a.C &&
                    grad_out.size(2) == 16 && grad_out.dtype() == torch::kFloat32,
                "grad_out must be float32 [N, C, 16]");
    torch::Tensor x = aligned16(node_features);
    torch::Tensor g = aligned16(grad_out.contiguous());
    torch::Tensor gpos = torch::empty({a.N, 3}, f32_like(x));
    if (a.N == 0) return gpos;
    const int64_t* ord = mace_order(order, a.N, x);
    const c10::DeviceGuard guard(x.device());
    const size_t wsb = batteries_mace_workspace_bytes(a.N, a.E, (int)a.C, 1);
    torch::Tensor ws = torch::empty({(int64_t)((wsb + 3) / 4)}, f32_like(x));
    check_status(batteries_mace_backward(cptr<float>(positions, "positions"), a.box,
                                         cptr<float>(x, "node_features"), cptr<float>(w1, "W1"),
                                         cptr<float>(b1, "b1"), cptr<float>(w2, "W2"),
                                         cptr<int64_t>(src, "src"), cptr<int64_t>(dst, "dst"),
                                         cptr<int64_t>(row_ptr, "row_ptr"), ord,
                                         cptr<int64_t>(rev, "rev"), cptr<float>(g, "grad_out"),
                                         mptr<float>(gpos, "grad_pos"), a.N, a.E, (int)a.C,
                                         (float)cutoff, ws.data_ptr(), wsb, current_stream(x)),
                 "mace_backward");
    return gpos;
}

}  // namespace

PYBIND11_MODULE(_batmobile, m) {
    namespace py = pybind11;
    m.doc() = "batmobile on MI355X: HIP kernels for equivariant message passing";
    m.def("spherical_harmonics", &spherical_harmonics, py::arg("edge_vectors"), py::arg("L_max"),
          "Real spherical harmonics Y_lm [N, (L_max+1)^2] of edge_vectors [N, 3], L_max in [0, 6]");
    m.def("spherical_harmonics_inplace", &spherical_harmonics_inplace, py::arg("edge_vectors"),
          py::arg("Y_lm"), py::arg("L_max"),
          "Compute spherical harmonics with pre-allocated output buffer");
    m.def("tensor_product_simple", &tensor_product_simple, py::arg("input1"), py::arg("input2"),
          "Simple 34-path CG tensor product [N,16] x [N,16] -> [N,16]");
    m.def("tensor_product", &tensor_product, py::arg("input1"), py::arg("input2"),
          py::arg("weights"),
          "Channel-weighted tensor product [N,C_in,16] x [N,16], W [34,C_in,C_out] -> [N,C_out,16]");
    m.def("get_tp_path_info", &get_tp_path_info,
          "Tensor product path info as [num_paths, 3] int32 (l1, l2, l_out)");
    m.def("get_tp_num_paths", &get_tp_num_paths, "Number of tensor product paths for L_max=3");
    m.def("spherical_harmonics_backward", &spherical_harmonics_backward, py::arg("edge_vectors"),
          py::arg("grad_Y_lm"), "Backward of spherical_harmonics w.r.t. edge_vectors");
    m.def("tensor_product_simple_backward", &tensor_product_simple_backward, py::arg("input1"),
          py::arg("input2"), py::arg("grad_output"), "(grad_input1, grad_input2)");
    m.def("tensor_product_backward", &tensor_product_backward, py::arg("input1"),
          py::arg("input2"), py::arg("weights"), py::arg("grad_output"),
          py::arg("needs_input1_grad") = true, py::arg("needs_input2_grad") = true,
          py::arg("needs_weights_grad") = true,
          "(grad_input1, grad_input2, grad_weights); skipped gradients are None");
    m.def("edge_index_to_csr", &edge_index_to_csr, py::arg("edge_index"), py::arg("N_atoms"),
          "COO edge_index [2, E] -> (row_ptr [N+1], col_idx [E]) grouped by target");
    m.def("fused_message_passing_simple", &fused_message_passing_simple,
          py::arg("node_features"), py::arg("edge_vectors"), py::arg("edge_index"),
          py::arg("row_ptr"), py::arg("col_idx"), "SH -> TP -> scatter_add in one kernel");
    m.def("fused_message_passing", &fused_message_passing, py::arg("node_features"),
          py::arg("edge_vectors"), py::arg("weights"), py::arg("row_ptr"), py::arg("col_idx"),
          "Fused message passing with dense channel-mixing weights [C_in, C_out]");
    m.def("fused_sh_tp_simple", &fused_sh_tp_simple, py::arg("edge_vectors"),
          py::arg("node_features"), py::arg("source_idx"),
          "Fused SH + simple TP -> messages [N_edges, C, 16]");
    // extensions
    m.def("spherical_harmonics_normalized", &spherical_harmonics_normalized,
          py::arg("edge_vectors"), py::arg("L_max"),
          "spherical_harmonics of v / max(|v|, 1e-10), normalisation fused");
    m.def("spherical_harmonics_normalized_backward", &spherical_harmonics_normalized_backward,
          py::arg("edge_vectors"), py::arg("grad_Y_lm"),
          "gradient of spherical_harmonics_normalized w.r.t. the raw vectors");
    m.def("sh_tp_scatter", &sh_tp_scatter, py::arg("edge_vectors"), py::arg("node_features"),
          py::arg("source_idx"), py::arg("row_ptr"), py::arg("perm") = py::none(),
          py::arg("normalize") = false,
          "Fused SH + simple TP + scatter-add over CSR rows (no messages tensor, no atomics)");
    m.def("weighted_tile_order", &weighted_tile_order, py::arg("order"), py::arg("row_ptr"),
          "Processing order for sh_tp_scatter_weighted: destinations grouped by edge count, "
          "each XCD's tiles by decreasing edge count");
    m.def("sh_tp_scatter_weighted", &sh_tp_scatter_weighted, py::arg("edge_vectors"),
          py::arg("node_features"), py::arg("weights"), py::arg("source_idx"), py::arg("row_ptr"),
          py::arg("perm") = py::none(), py::arg("order") = py::none(), py::arg("normalize") = true,
          "Fused SH + weighted TP (W [34, C_in, C_out]) + scatter-add over CSR rows");
    m.def("neighbor_graph", &neighbor_graph, py::arg("positions"), py::arg("cell"),
          py::arg("cutoff"), py::arg("self_loops") = false,
          "neighbor list in the message-passing layout: (src = j, dst = i, pos[i] - pos[j], row_offsets, spatial_order)");
    m.def("neighbor_list", &neighbor_list, py::arg("positions"), py::arg("cell"),
          py::arg("cutoff"), py::arg("self_loops") = false, py::arg("row_capacity") = 0,
          "Cell-list PBC neighbor list -> (edge_index [2,E] int64, edge_vectors [E,3], "
          "row_offsets); up to 8192 atoms in three kernels and a scan (row_capacity: entries "
          "per atom of its slab, 0 = from the density; < 0 takes the general passes)");
    m.def("spatial_order", &spatial_order, py::arg("positions"), py::arg("cell"),
          "Atoms sorted by the Morton code of their cell (2^b cells per axis, the largest "
          "b <= 5 with 8^b <= N)");
    m.def("neighbor_graph_capacity", &neighbor_graph_capacity, py::arg("positions"),
          py::arg("cell"), py::arg("cutoff"), py::arg("self_loops"), py::arg("capacity"),
          "neighbor_graph with arrays of `capacity` edges and no host synchronisation: "
          "(src, dst, edge_vectors, row_offsets, order, overflow); the edge count is "
          "row_offsets[-1] on the device, overflow [1] is 1 (and every row empty) when it "
          "exceeded the capacity");
    m.def("graph_build", &graph_build, py::arg("positions"), py::arg("cell"), py::arg("cutoff"),
          py::arg("self_loops"), py::arg("C"), py::arg("max_edges") = -1,
          py::arg("row_capacity") = 0,
          "batmobile.Graph's build in four kernels (None outside its limits): (src, dst, "
          "edge_vectors, row_offsets, order, row_ptr_s, edge_perm, row_dst, n_blocks, "
          "rows_per_block, overflow or None)");
    m.def("mp_schedule", &mp_schedule, py::arg("row_ptr"), py::arg("order"), py::arg("C"),
          py::arg("col_perm") = py::none(), py::arg("num_edges") = -1,
          "Spatial processing schedule for sh_tp_scatter_scheduled: "
          "(row_ptr_s, edge_perm, row_dst, n_blocks, rows_per_block); num_edges = row_ptr[-1] "
          "when the caller knows it (saves a host sync)");
    m.def("sh_tp_scatter_scheduled", &sh_tp_scatter_scheduled, py::arg("edge_vectors"),
          py::arg("node_features"), py::arg("source_idx"), py::arg("row_ptr_s"),
          py::arg("edge_perm"), py::arg("row_dst"), py::arg("n_blocks"),
          py::arg("rows_per_block"), py::arg("N_dst"), py::arg("normalize") = false,
          py::arg("channel_split") = false,
          "sh_tp_scatter processed in the order of an mp_schedule (same result); channel_split: "
          "XCD halves take channel halves (graphs whose sources have no spatial order)");
    m.def("gemm_f32", &gemm_f32, py::arg("A"), py::arg("B"), py::arg("trans_b") = false,
          "C = A @ B (or A @ B.T) on MFMA, fp32 (extension)");
    m.def("mace_reverse_edges", &mace_reverse_edges, py::arg("row_ptr"), py::arg("src"),
          "index of every edge's reverse in a symmetric destination-grouped edge list (extension)");
    m.def("mace_forward", &mace_forward, py::arg("positions"), py::arg("cell"),
          py::arg("node_features"), py::arg("W1"), py::arg("b1"), py::arg("W2"), py::arg("src"),
          py::arg("dst"), py::arg("row_ptr"), py::arg("cutoff"), py::arg("order") = py::none(),
          "MACE-style layer with per-edge radial weights, forward (extension; one fused kernel, "
          "the per-edge weights stay on chip); order [N], a permutation of 0..N-1, is the "
          "processing order of the destinations (results do not depend on it)");
    m.def("mace_backward", &mace_backward, py::arg("positions"), py::arg("cell"),
          py::arg("node_features"), py::arg("W1"), py::arg("b1"), py::arg("W2"), py::arg("src"),
          py::arg("dst"), py::arg("row_ptr"), py::arg("rev"), py::arg("grad_out"),
          py::arg("cutoff"), py::arg("order") = py::none(),
          "gradient of the MACE-style layer w.r.t. positions (extension); order as for "
          "mace_forward");
    m.def("selftest_mfma_16x16x4", &selftest_mfma_16x16x4, py::arg("A"), py::arg("B"),
          "D = A @ B through one v_mfma_f32_16x16x4f32 (lane-layout self test)");
    m.def("selftest_mfma_4x4x1_bcast", &selftest_mfma_4x4x1_bcast, py::arg("A"), py::arg("B"),
          "D[k, l, r]: one v_mfma_f32_4x4x1_16b_f32 with A of block k broadcast (layout check)");
}
