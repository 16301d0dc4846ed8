// gpu_cli: the reference's GPU search CLI (src/gpu_cli.cu:353-492) on the MI355X.
//
// Reads one JSON object from stdin:
//   {"data":   {"graph", "base", "query", "gt", "codebook"?},
//    "search": {"mode", "K", "topk_size", "filter_capacity", "max_iterations", "reset_interval"}}
// loads the files, uploads the index through the C-ABI (include/bs_hip.h), runs one
// warm-up and 5 timed searches and prints the reference's line protocol:
//   data: N points, dim=D, degree=R, queries=Q, entry=E
//   search: mode=M K=K
//     time: X ms  qps: Y            (kernel time per run, HIP events)
//     duplicates: ...               (only when some query returned an id twice)
//   recall@K: R
// Exit status 1 on a configuration or input error, with the message on stderr.
#include "bs_hip.h"
#include "bs_host.h"
#include "cli_config.hpp"
#include "json_lite.hpp"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <iostream>
#include <iterator>
#include <string>
#include <vector>

namespace {

struct Buf {
    void* p = nullptr;
    ~Buf() { bs_host_free(p); }
};

int die(const std::string& m) {
    std::cerr << m << std::endl;
    return 1;
}

}  // namespace

int main() {
    const std::string text((std::istreambuf_iterator<char>(std::cin)), std::istreambuf_iterator<char>());
    jsonl::Value j;
    try {
        j = jsonl::parse(text);
    } catch (const std::exception& e) {
        return die(std::string("JSON parse error: ") + e.what());
    }
    try {
        cli::DataFiles files;
        std::string err = cli::read_data(j, files);
        if (!err.empty()) return die(err);
        const std::string &graph_file = files.graph, &base_file = files.base, &query_file = files.query,
                          &gt_file = files.gt, &codebook_file = files.codebook;

        Buf eb, vb, qb, gb;
        uint64_t n = 0, nv = 0, nq = 0, ngt = 0;
        uint32_t degree = 0, dim = 0, qdim = 0, gt_k = 0;
        if (bs_read_graph(graph_file.c_str(), reinterpret_cast<uint32_t**>(&eb.p), &n, &degree))
            return die(bs_host_last_error());
        std::cout << "Loaded graph: " << n << " nodes, degree " << degree << " from " << graph_file << "\n";
        if (bs_read_vecs(base_file.c_str(), 0, &vb.p, &nv, &dim)) return die(bs_host_last_error());
        if (nv != n) return die("base vectors (" + std::to_string(nv) + ") do not match graph nodes (" +
                                std::to_string(n) + ")");
        std::cout << "Loaded vectors: " << n << " x " << dim << " from " << base_file << "\n";
        if (bs_read_vecs(query_file.c_str(), 0, &qb.p, &nq, &qdim)) return die(bs_host_last_error());
        if (qdim != dim && nq) return die("query dim does not match base dim");
        if (bs_read_vecs(gt_file.c_str(), 1, &gb.p, &ngt, &gt_k)) return die(bs_host_last_error());
        if (ngt < nq) return die("ground truth has fewer rows than queries");

        const float* vecs = static_cast<const float*>(vb.p);
        const uint32_t* edges = static_cast<const uint32_t*>(eb.p);
        bs_index ix = nullptr;
        if (bs_index_create(vecs, edges, n, dim, degree, &ix)) return die(bs_last_error());
        uint32_t entry = 0;  // compute_entry_point (src/gpu_cli.cu:55-83), on the device
        if (bs_index_entry_point(ix, &entry)) return die(bs_last_error());
        std::cout << "data: " << n << " points, dim=" << dim << ", degree=" << degree << ", queries=" << nq
                  << ", entry=" << entry << std::endl;

        cli::SearchSettings ss;
        if (!(err = cli::read_search_head(j, ss)).empty()) return die(err);
        const std::string& mode = ss.mode;
        const int K = ss.K;
        std::cout << "search: mode=" << mode << " K=" << K << std::endl;
        if (!(err = cli::read_search_rest(j, !codebook_file.empty(), ss)).empty()) return die(err);
        bs_search_cfg cfg = ss.cfg;
        cfg.entry_point = entry;
        if (cfg.mode == BS_RABITQ) {
            uint32_t cb_entry = 0, pdim = 0;
            Buf cb, fb, sb;
            if (bs_read_codebook(codebook_file.c_str(), n, dim, degree, &cb_entry,
                                 reinterpret_cast<uint32_t**>(&cb.p), reinterpret_cast<float**>(&fb.p),
                                 reinterpret_cast<float**>(&sb.p), &pdim))
                return die(bs_host_last_error());
            std::cout << "Loaded rabitq codebook: " << n << " nodes, dim=" << dim << ", degree=" << degree
                      << ", padded_dim=" << pdim << " (entry=" << cb_entry << ")\n";
            if (bs_index_attach_rabitq(ix, static_cast<uint32_t*>(cb.p), static_cast<float*>(fb.p),
                                       static_cast<float*>(sb.p), pdim))
                return die(bs_last_error());
            cfg.entry_point = (cb_entry != 0xFFFFFFFFu) ? cb_entry : entry;
        }

        const float* queries = static_cast<const float*>(qb.p);
        std::vector<uint32_t> results(nq * static_cast<uint64_t>(K), 0xFFFFFFFFu);
        bs_stats st{};
        // one warm-up (the reference has none, so its first run includes launch set-up)
        if (bs_search(ix, &cfg, queries, nq, results.data(), nullptr, &st)) return die(bs_last_error());
        constexpr int NRUNS = 5;
        double kms = 0.0;
        for (int r = 0; r < NRUNS; ++r) {
            if (bs_search(ix, &cfg, queries, nq, results.data(), nullptr, &st)) return die(bs_last_error());
            kms += st.kernel_ms;
        }
        const double ms = kms / NRUNS;
        std::cout << "  time: " << ms << " ms  qps: " << (ms > 0 ? nq / (ms / 1000.0) : 0.0) << std::endl;

        // recall (src/gpu_cli.cu:28-51): reads gt_k columns per query
        std::vector<int32_t> gt(static_cast<const int32_t*>(gb.p), static_cast<const int32_t*>(gb.p) + nq * gt_k);
        uint64_t dups = 0;
        const double rec = nq ? bs_recall(results.data(), nq, static_cast<uint32_t>(K), gt.data(), gt_k, &dups) : 0.0;
        if (dups > 0)
            std::cout << "  duplicates: " << dups << " total (" << static_cast<double>(dups) / nq << " avg/query)"
                      << std::endl;
        std::cout << "recall@" << K << ": " << rec << std::endl;
        bs_index_destroy(ix);
        return 0;
    } catch (const std::exception& e) {
        return die(e.what());
    }
}
