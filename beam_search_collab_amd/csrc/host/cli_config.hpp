// gpu_cli's configuration: the JSON keys, defaults and checks of the reference CLI
// (src/gpu_cli.cu:353-477), in the two steps the CLI takes -- the data files first, the
// search settings after the files are loaded -- so that cli_config_check (the sanitizer
// harness) runs the same code on any text.  Every function returns "" or the error
// message the CLI prints before exiting with status 1.
#pragma once
#include "bs_hip.h"
#include "json_lite.hpp"

#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <string>

namespace cli {

struct DataFiles {
    std::string graph, base, query, gt, codebook;
};

struct SearchSettings {
    std::string mode = "base";
    int K = 100;
    bs_search_cfg cfg{};
};

// A JSON number as an integer in [lo, hi], truncated toward zero as the reference's
// json::value<int> conversion does.  Non-finite and out-of-range numbers are an error here
// (the conversion itself would be undefined).
inline std::string int_value(const jsonl::Value& obj, const char* key, int64_t dflt, int64_t lo, int64_t hi,
                             int64_t& out) {
    if (!obj.has(key)) {
        out = dflt;
        return "";
    }
    const jsonl::Value& v = obj.at(key);
    if (v.kind != jsonl::Value::Number) return std::string("\"") + key + "\" must be a number";
    const double t = std::trunc(v.num);
    if (!std::isfinite(t) || t < static_cast<double>(lo) || t > static_cast<double>(hi))
        return std::string("\"") + key + "\" is out of range [" + std::to_string(lo) + ", " + std::to_string(hi) + "]";
    out = static_cast<int64_t>(t);
    return "";
}

inline std::string string_value(const jsonl::Value& obj, const char* key, bool required, std::string& out) {
    if (!obj.has(key)) return required ? std::string("Missing \"") + key + "\" key" : std::string();
    const jsonl::Value& v = obj.at(key);
    if (v.kind != jsonl::Value::String) return std::string("\"") + key + "\" must be a string";
    out = v.str;
    return "";
}

// The legacy modes, then the data block (src/gpu_cli.cu:364-394).
inline std::string read_data(const jsonl::Value& j, DataFiles& d) {
    if (j.kind != jsonl::Value::Object) return "the configuration must be a JSON object";
    if (j.has("search") && j.at("search").kind == jsonl::Value::Object && j.at("search").has("mode")) {
        const jsonl::Value& m = j.at("search").at("mode");
        if (m.kind == jsonl::Value::String && m.str.rfind("sophia_", 0) == 0)
            return "mode " + m.str + ": the legacy sophia_* stack is not part of this build";
    }
    if (!j.has("data")) return "Missing \"data\" key";
    const jsonl::Value& jd = j.at("data");
    if (jd.kind != jsonl::Value::Object) return "\"data\" must be an object";
    std::string e;
    if (!(e = string_value(jd, "graph", true, d.graph)).empty()) return e;
    if (!(e = string_value(jd, "base", true, d.base)).empty()) return e;
    if (!(e = string_value(jd, "query", true, d.query)).empty()) return e;
    if (!(e = string_value(jd, "gt", true, d.gt)).empty()) return e;
    return string_value(jd, "codebook", false, d.codebook);
}

// The search block's mode and K (printed by the CLI before anything is checked further).
inline std::string read_search_head(const jsonl::Value& j, SearchSettings& s) {
    if (!j.has("search")) return "Missing \"search\" key";
    const jsonl::Value& js = j.at("search");
    if (js.kind != jsonl::Value::Object) return "\"search\" must be an object";
    std::string e = string_value(js, "mode", false, s.mode);
    if (!e.empty()) return e;
    int64_t K = 0;
    if (!(e = int_value(js, "K", 100, INT32_MIN, INT32_MAX, K)).empty()) return e;
    s.K = static_cast<int>(K);
    return "";
}

// The rest of the search block and the mode (src/gpu_cli.cu:396-477): cfg is filled except
// for the entry point, which the CLI takes from the index or the codebook.
inline std::string read_search_rest(const jsonl::Value& j, bool have_codebook, SearchSettings& s) {
    if (s.K <= 0) return "K must be positive";
    const jsonl::Value& js = j.at("search");
    bs_search_cfg& cfg = s.cfg;
    cfg = bs_search_cfg{};
    cfg.K = static_cast<uint32_t>(s.K);
    int64_t v = 0;
    std::string e;
    if (!(e = int_value(js, "topk_size", 256, 0, UINT32_MAX, v)).empty()) return e;
    cfg.topk_size = static_cast<uint32_t>(v);
    if (!(e = int_value(js, "filter_capacity", 1024, 0, UINT32_MAX, v)).empty()) return e;
    cfg.filter_capacity = static_cast<uint32_t>(v);
    if (!(e = int_value(js, "max_iterations", 1024, INT32_MIN, INT32_MAX, v)).empty()) return e;
    cfg.max_iterations = static_cast<int32_t>(v);
    if (!(e = int_value(js, "reset_interval", 16, INT32_MIN, INT32_MAX, v)).empty()) return e;
    cfg.reset_interval = static_cast<int32_t>(v);
    cfg.queries_per_group = 1;
    const std::string& mode = s.mode;
    if (mode == "rabitq") {
        if (!have_codebook) return "rabitq mode requires \"codebook\" in data config";
        cfg.mode = BS_RABITQ;
        cfg.reset_interval = 0;
        return "";
    }
    if (cfg.topk_size < static_cast<uint32_t>(s.K))
        return "topk_size (" + std::to_string(cfg.topk_size) + ") must be >= K (" + std::to_string(s.K) + ")";
    if (mode == "base") {
        cfg.mode = BS_BASE;
        return "";
    }
    if (mode.size() >= 5 && (mode.rfind("warp", 0) == 0 || mode.rfind("bwarp", 0) == 0)) {
        const bool bloom = mode[0] == 'b';
        const std::string ny = mode.substr(bloom ? 5 : 4);
        if (ny != "1" && ny != "2" && ny != "4" && ny != "8") return "Unknown mode: " + mode;
        cfg.mode = bloom ? BS_GROUP_BLOOM : BS_GROUP;
        cfg.queries_per_group = static_cast<uint32_t>(std::atoi(ny.c_str()));
        return "";
    }
    return "Unknown mode: " + mode;
}

}  // namespace cli
