// SPDX-License-Identifier: MIT
//
// beamgrad_amd._C: owner of the torch.ops.beamgrad namespace. It defines the
// seven operator schemas of the reference (python/csrc/cpu_ops.cpp:582-608,
// the text kept identical so either library's kernels serve the other's
// definitions) and registers no kernel: the HIP kernels come from
// beamgrad_amd._C_hip (torch_ops.cpp), which only adds implementations and
// its own operators to the namespace and so also loads beside the
// reference's _C in place of its _C_cuda.
//
// beamgrad_amd's Python front end loads this module only when no other
// library has defined the namespace yet: torch allows one definition
// (TORCH_LIBRARY) per namespace and ends the process on a second one.
#include <Python.h>

#include <torch/library.h>

TORCH_LIBRARY(beamgrad, m) {
    m.def(
        "decode(Tensor log_probs, Tensor? steps, int eos_token, int min_length, float length_penalty_alpha, "
        "Tensor? banned_tokens, int no_repeat_ngram_size, float repetition_penalty, bool validate) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def(
        "final_scores_backward(Tensor grad_final, Tensor parents, Tensor tokens, Tensor lengths, "
        "Tensor from_logprob, Tensor? steps, int vocab_size, float length_penalty_alpha) -> Tensor");
    m.def("length_penalty(Tensor lengths, float length_penalty_alpha) -> Tensor");
    m.def(
        "final_scores_path_gradient(Tensor grad_final, Tensor parents, Tensor tokens, Tensor lengths, "
        "Tensor from_logprob, Tensor? steps, int vocab_size, float length_penalty_alpha) -> Tensor");
    m.def(
        "decode_step(Tensor log_probs, Tensor raw_scores, Tensor lengths, Tensor finished, Tensor prefixes, "
        "int eos_token, int min_length, float length_penalty_alpha, Tensor? banned_tokens, int no_repeat_ngram_size, "
        "float repetition_penalty, bool validate, int[] extra_eos=[]) -> "
        "(Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor)");
    m.def(
        "decode_ex(Tensor inputs, bool from_logits, Tensor? steps, int eos_token, int min_length, "
        "float length_penalty_alpha, Tensor? banned_tokens, int no_repeat_ngram_size, float repetition_penalty, "
        "bool validate, int[] extra_eos=[]) -> (Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, "
        "Tensor)");
    m.def(
        "decode_backward(Tensor? grad_final_scores, Tensor? grad_final_raw_scores, Tensor? grad_scores, "
        "Tensor? grad_raw_scores, Tensor parents, Tensor tokens, Tensor lengths, Tensor from_logprob, Tensor? steps, "
        "int vocab_size, float length_penalty_alpha, Tensor? logits, Tensor? row_lse) -> Tensor");
}

PyMODINIT_FUNC PyInit__C(void) {
    static PyModuleDef module = {
        PyModuleDef_HEAD_INIT, "_C", "defines the torch.ops.beamgrad operator schemas (no kernels)", -1, nullptr,
    };
    return PyModule_Create(&module);
}
