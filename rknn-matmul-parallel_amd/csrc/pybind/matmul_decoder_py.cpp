// matmul_decoder_py.cpp — the `matmul_decoder` Python module over the C ABI.
//
// Same Python surface as the reference module (reference:
// src/pybind_matmul_decoder.cpp:294-386): class MatmulDecoder(model_dir,
// max_seq_len=4096, quant_type="int4", exec_mode="dual_core",
// disable_npu_lm_head=False) with step, prefill, prefill_batch,
// step_get_token, clear_kv_cache, generate, seq_len, config, stats; module
// functions config_qwen3_0_6b*, __version__ "1.0.0".  Differences, on
// purpose: embeddings are taken as C-contiguous float32 (any input is
// converted) and must hold hidden_dim values per row; step() raises when the
// C call fails instead of returning an unfilled buffer; step_get_token skips
// the logits copy it never returns; generate() feeds the last prompt token
// and then each sampled token (the reference fed token -1, which the C step
// rejects).
#include <pybind11/functional.h>
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "matmul_decoder.h"
#include "mdx_ext.h"

namespace py = pybind11;

using FArray = py::array_t<float, py::array::c_style | py::array::forcecast>;

namespace {

QuantizationType parse_quant(const std::string& q) {
    if (q == "fp16") return QUANT_FP16;
    if (q == "int8") return QUANT_INT8;
    if (q == "int4_g128") return QUANT_INT4_G128;
    return QUANT_INT4;
}

py::dict config_dict(const MatmulDecoderConfig& c, const char* exec_name) {
    return py::dict(py::arg("name") = std::string(c.name ? c.name : ""),
                    py::arg("hidden_dim") = c.hidden_dim, py::arg("num_q_heads") = c.num_q_heads,
                    py::arg("num_kv_heads") = c.num_kv_heads, py::arg("head_dim") = c.head_dim,
                    py::arg("ffn_dim") = c.ffn_dim, py::arg("num_layers") = c.num_layers,
                    py::arg("vocab_size") = c.vocab_size, py::arg("has_qk_norm") = c.has_qk_norm,
                    py::arg("exec_mode") = exec_name);
}

class PyMatmulDecoder {
public:
    PyMatmulDecoder(const std::string& model_dir, int max_seq_len, const std::string& quant_type,
                    const std::string& exec_mode, bool disable_npu_lm_head) {
        MatmulDecoderConfig cfg;
        const std::string cfg_path = model_dir + "/config.json";
        if (matmul_decoder_load_config(cfg_path.c_str(), &cfg) != 0)
            throw std::runtime_error("Failed to load config.json from " + model_dir);
        cfg.exec_mode = exec_mode == "single_core" ? EXEC_SINGLE_CORE : EXEC_DUAL_CORE;
        cfg.max_seq_len = max_seq_len;
        cfg.disable_npu_lm_head = disable_npu_lm_head ? 1 : 0;
        {
            py::gil_scoped_release nogil;
            ctx_ = matmul_decoder_create(model_dir.c_str(), &cfg, parse_quant(quant_type), max_seq_len);
        }
        if (!ctx_) throw std::runtime_error("Failed to create MatmulDecoder from " + model_dir);
        cfg_ = cfg;
    }

    ~PyMatmulDecoder() { matmul_decoder_destroy(ctx_); }

    PyMatmulDecoder(const PyMatmulDecoder&) = delete;
    PyMatmulDecoder& operator=(const PyMatmulDecoder&) = delete;

    const float* row_ptr(const FArray& a) const {
        if (a.size() < cfg_.hidden_dim)
            throw std::invalid_argument("embedding must hold hidden_dim=" +
                                        std::to_string(cfg_.hidden_dim) + " values");
        return a.data();
    }

    py::array_t<float> step(int token_id, py::object embedding) {
        FArray emb;
        const float* ep = nullptr;
        if (!embedding.is_none()) {
            emb = embedding.cast<FArray>();
            ep = row_ptr(emb);
        }
        py::array_t<float> logits(cfg_.vocab_size);
        float* lp = logits.mutable_data();
        int rc;
        {
            py::gil_scoped_release nogil;
            rc = matmul_decoder_step(ctx_, token_id, ep, lp);
        }
        if (rc < 0) throw std::runtime_error("step failed with error code " + std::to_string(rc));
        return logits;
    }

    void prefill_batch(py::object embeddings) {
        FArray a = embeddings.cast<FArray>();
        if (a.ndim() != 2) throw std::runtime_error("prefill_batch: embeddings must be 2D [M, hidden_dim]");
        if (a.shape(1) != cfg_.hidden_dim)
            throw std::runtime_error("prefill_batch: second dimension must be hidden_dim");
        const int M = (int)a.shape(0);
        int rc;
        {
            py::gil_scoped_release nogil;
            rc = matmul_decoder_prefill_batch(ctx_, a.data(), M);
        }
        if (rc != 0) throw std::runtime_error("prefill_batch failed with error code " + std::to_string(rc));
    }

    void prefill(int token_id, py::object embedding) {
        const float* ep = nullptr;
        FArray emb;
        if (!embedding.is_none()) {
            emb = embedding.cast<FArray>();
            if (emb.ndim() == 2) {
                prefill_batch(emb);
                return;
            }
            ep = row_ptr(emb);
        }
        py::gil_scoped_release nogil;
        matmul_decoder_step(ctx_, token_id, ep, nullptr);
    }

    int step_get_token(int token_id, py::object embedding) {
        FArray emb;
        const float* ep = nullptr;
        if (!embedding.is_none()) {
            emb = embedding.cast<FArray>();
            ep = row_ptr(emb);
        }
        py::gil_scoped_release nogil;
        return mdx_step_token(ctx_, token_id, ep);
    }

    // One step, then a draw on the device (matmul_decoder_step_sample); u is
    // the caller's uniform in [0,1].  Not in the reference module.
    int step_sample(int token_id, float u, int top_k, float top_p, float temperature,
                    float repeat_penalty, std::vector<int> repeat_tokens, py::object embedding) {
        FArray emb;
        const float* ep = nullptr;
        if (!embedding.is_none()) {
            emb = embedding.cast<FArray>();
            ep = row_ptr(emb);
        }
        SamplingParams p = sampling_params_greedy();
        p.top_k = top_k;
        p.top_p = top_p;
        p.temperature = temperature;
        p.repeat_penalty = repeat_penalty;
        p.repeat_tokens = repeat_tokens.empty() ? nullptr : repeat_tokens.data();
        p.n_repeat_tokens = (int)repeat_tokens.size();
        int tok;
        {
            py::gil_scoped_release nogil;
            tok = matmul_decoder_step_sample(ctx_, token_id, ep, &p, u, nullptr);
        }
        if (tok < 0) throw std::runtime_error("step_sample failed (" + std::to_string(tok) + ")");
        return tok;
    }

    void clear_kv_cache() { matmul_decoder_clear_kv_cache(ctx_); }

    int seq_len() const { return matmul_decoder_get_seq_len(ctx_); }

    py::dict config() const {
        return py::dict(py::arg("name") = std::string(cfg_.name ? cfg_.name : ""),
                        py::arg("hidden_dim") = cfg_.hidden_dim,
                        py::arg("num_q_heads") = cfg_.num_q_heads,
                        py::arg("num_kv_heads") = cfg_.num_kv_heads,
                        py::arg("head_dim") = cfg_.head_dim, py::arg("ffn_dim") = cfg_.ffn_dim,
                        py::arg("num_layers") = cfg_.num_layers,
                        py::arg("vocab_size") = cfg_.vocab_size,
                        py::arg("max_seq_len") = cfg_.max_seq_len, py::arg("rms_eps") = cfg_.rms_eps,
                        py::arg("rope_theta") = cfg_.rope_theta,
                        py::arg("tie_word_embeddings") = cfg_.tie_word_embeddings,
                        py::arg("has_qk_norm") = cfg_.has_qk_norm,
                        py::arg("exec_mode") = cfg_.exec_mode == EXEC_DUAL_CORE ? "dual_core" : "single_core");
    }

    py::dict stats() const {
        MatmulDecoderStats s = {};
        matmul_decoder_get_stats(ctx_, &s);
        return py::dict(py::arg("total_ms") = s.total_ms, py::arg("matmul_ms") = s.matmul_ms,
                        py::arg("rebind_ms") = s.rebind_ms, py::arg("convert_ms") = s.convert_ms,
                        py::arg("cpu_ops_ms") = s.cpu_ops_ms, py::arg("lm_head_ms") = s.lm_head_ms,
                        py::arg("n_steps") = s.n_steps);
    }

    std::vector<int> generate(const std::vector<int>& prompt_tokens, int max_new_tokens, int top_k,
                              float top_p, float temperature, float repeat_penalty,
                              py::object callback) {
        std::vector<int> out;
        if (prompt_tokens.empty()) return out;
        SamplingParams params = sampling_params_greedy();
        params.top_k = top_k;
        params.top_p = top_p;
        params.temperature = temperature;
        params.repeat_penalty = repeat_penalty;
        for (size_t i = 0; i + 1 < prompt_tokens.size(); i++) {
            py::gil_scoped_release nogil;
            matmul_decoder_step(ctx_, prompt_tokens[i], nullptr, nullptr);
        }
        std::vector<float> logits((size_t)cfg_.vocab_size);
        int tok = prompt_tokens.back();
        for (int i = 0; i < max_new_tokens; i++) {
            int next;
            {
                py::gil_scoped_release nogil;
                next = matmul_decoder_step(ctx_, tok, nullptr, logits.data());
            }
            if (next < 0) break;
            if (top_k > 1) next = matmul_sample_token(logits.data(), cfg_.vocab_size, &params);
            out.push_back(next);
            if (!callback.is_none()) callback(next);
            tok = next;
        }
        return out;
    }

private:
    MatmulDecoderContext* ctx_ = nullptr;
    MatmulDecoderConfig cfg_{};
};

}  // namespace

PYBIND11_MODULE(matmul_decoder, m) {
    m.doc() = "Matmul decoder on AMD Instinct MI355X (gfx950)";

    py::class_<PyMatmulDecoder>(m, "MatmulDecoder")
        .def(py::init<const std::string&, int, const std::string&, const std::string&, bool>(),
             py::arg("model_dir"), py::arg("max_seq_len") = 4096, py::arg("quant_type") = "int4",
             py::arg("exec_mode") = "dual_core", py::arg("disable_npu_lm_head") = false)
        .def("step", &PyMatmulDecoder::step, py::arg("token_id"), py::arg("embedding") = py::none(),
             "Run one decoding step, return logits")
        .def("prefill", &PyMatmulDecoder::prefill, py::arg("token_id"), py::arg("embedding") = py::none(),
             "Run one prefill step (fills the KV cache, no lm_head); a 2D embedding routes to "
             "prefill_batch")
        .def("prefill_batch", &PyMatmulDecoder::prefill_batch, py::arg("embeddings"),
             "Batch prefill of M tokens, embeddings [M, hidden_dim]")
        .def("step_get_token", &PyMatmulDecoder::step_get_token, py::arg("token_id"),
             py::arg("embedding") = py::none(), "Run one decoding step, return the greedy token")
        .def("step_sample", &PyMatmulDecoder::step_sample, py::arg("token_id"), py::arg("u"),
             py::arg("top_k") = 40, py::arg("top_p") = 1.0f, py::arg("temperature") = 1.0f,
             py::arg("repeat_penalty") = 1.0f, py::arg("repeat_tokens") = std::vector<int>(),
             py::arg("embedding") = py::none(),
             "One decoding step, then top-k/top-p sampling on the device with uniform u in [0,1]")
        .def("clear_kv_cache", &PyMatmulDecoder::clear_kv_cache, "Clear the KV cache")
        .def("generate", &PyMatmulDecoder::generate, py::arg("prompt_tokens"),
             py::arg("max_new_tokens") = 128, py::arg("top_k") = 1, py::arg("top_p") = 1.0f,
             py::arg("temperature") = 1.0f, py::arg("repeat_penalty") = 1.0f,
             py::arg("callback") = py::none(), "Generate tokens autoregressively")
        .def_property_readonly("seq_len", &PyMatmulDecoder::seq_len, "Current sequence length")
        .def_property_readonly("config", &PyMatmulDecoder::config, "Model configuration")
        .def_property_readonly("stats", &PyMatmulDecoder::stats, "Performance statistics")
        .def("__repr__", [](const PyMatmulDecoder&) { return "<MatmulDecoder>"; });

    m.def("config_qwen3_0_6b", []() { return config_dict(matmul_decoder_config_qwen3_0_6b(), "dual_core"); },
          "Default config for Qwen3-0.6B (dual-core)");
    m.def("config_qwen3_0_6b_single_core",
          []() { return config_dict(matmul_decoder_config_qwen3_0_6b_single_core(), "single_core"); },
          "Default config for Qwen3-0.6B (single-core)");
    m.attr("__version__") = "1.0.0";
}
