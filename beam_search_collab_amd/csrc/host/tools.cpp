// build_graph / build_rabitq / gen_data / compute_gt command-line tools (one binary per
// tool, selected at compile time with -DBS_TOOL=...).
//   build_graph  --base B.fvecs --graph G.bin [--degree 32] [--beam-width 128] [--alpha 2.0]
//                [--metric l2] [--seed 1234] [--threads N] [--fast] [--device]
//                (flags of src/build_graph.cpp:210-256; --fast uses vectorized distances,
//                --device builds the same graph as the default on the GPU)
//   build_rabitq -base B.fvecs -graph G.bin -out CB.bin [-seed 12345] [-device]
//                (flags of src/build_rabitq.cpp:103-120; -device: the same codebook from the GPU)
//   gen_data     --out-base B.fvecs --out-query Q.fvecs --n N --nq Q --dim D
//                [--kind mixture|normalized] [--centres 64] [--lo 0] [--hi 128] [--sigma 12]
//   compute_gt   --base B.fvecs --query Q.fvecs --out GT.ivecs [--k 100]
//   replicate_queries <input.fvecs|ivecs> <output> <repeats> <fvecs|ivecs>
//                (positional arguments of src/replicate_queries.cpp:10-24; writes the input
//                rows `repeats` times in order, for larger query batches)
#include "bs_host.h"
#if BS_TOOL == 1 || BS_TOOL == 2
#include "bs_hip.h"
#endif

#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <iostream>
#include <map>
#include <string>
#include <vector>

namespace {

std::map<std::string, std::string> args(int argc, char** argv, const std::vector<std::string>& flags) {
    std::map<std::string, std::string> a;
    for (int i = 1; i < argc; ++i) {
        std::string k = argv[i];
        bool is_flag = false;
        for (const auto& f : flags) is_flag = is_flag || f == k;
        if (is_flag) {
            a[k] = "1";
        } else if (i + 1 < argc) {
            a[k] = argv[++i];
        } else {
            throw std::runtime_error("Missing value for argument: " + k);
        }
    }
    return a;
}

std::string get(const std::map<std::string, std::string>& a, const std::string& k, const std::string& d) {
    auto it = a.find(k);
    return it == a.end() ? d : it->second;
}

struct Buf {
    void* p = nullptr;
    ~Buf() { bs_host_free(p); }
};

double now() { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); }

}  // namespace

int main(int argc, char** argv) {
    try {
#if BS_TOOL == 1
        auto a = args(argc, argv, {"--fast", "--device", "--help"});
        if (a.count("--help")) {
            std::cout << "Usage: build_graph --base base.fvecs --graph graph.bin [--degree 32] [--beam-width 128]"
                         " [--alpha 2.0] [--metric l2] [--seed 1234] [--threads N] [--fast] [--device]\n";
            return 0;
        }
        const std::string base = get(a, "--base", ""), graph = get(a, "--graph", "");
        if (base.empty()) throw std::runtime_error("Missing required argument: --base");
        if (graph.empty()) throw std::runtime_error("Missing required argument: --graph");
        if (get(a, "--metric", "l2") != "l2") throw std::runtime_error("Unsupported metric: only l2 is built here");
        const int degree = std::stoi(get(a, "--degree", "32")), beam = std::stoi(get(a, "--beam-width", "128"));
        const double alpha = std::stod(get(a, "--alpha", "2.0"));
        const uint32_t seed = static_cast<uint32_t>(std::stoul(get(a, "--seed", "1234")));
        Buf v;
        uint64_t n = 0;
        uint32_t dim = 0;
        if (bs_read_vecs(base.c_str(), 0, &v.p, &n, &dim)) throw std::runtime_error(bs_host_last_error());
        std::cout << "Building Vamana graph: n=" << n << " dim=" << dim << " degree=" << degree
                  << " beam_width=" << beam << " alpha=" << alpha << " metric=l2\n";
        std::vector<uint32_t> edges(n * static_cast<uint64_t>(degree));
        const double t0 = now();
        if (a.count("--device")) {
            if (bs_build_vamana_device(static_cast<float*>(v.p), n, dim, degree, beam, static_cast<float>(alpha), seed,
                                       edges.data(), 1))
                throw std::runtime_error(bs_last_error());
        } else if (bs_build_vamana(static_cast<float*>(v.p), n, dim, degree, beam, static_cast<float>(alpha), seed,
                                   a.count("--fast") ? 0 : 1, std::stoi(get(a, "--threads", "0")), edges.data(), 1)) {
            throw std::runtime_error(bs_host_last_error());
        }
        if (bs_write_graph(graph.c_str(), edges.data(), n, degree)) throw std::runtime_error(bs_host_last_error());
        std::cout << "Wrote graph to " << graph << "\nTotal build time: " << now() - t0 << "s\n";
#elif BS_TOOL == 2
        auto a = args(argc, argv, {"-device"});
        const std::string base = get(a, "-base", ""), graph = get(a, "-graph", ""), out = get(a, "-out", "");
        if (base.empty() || graph.empty() || out.empty()) {
            std::cerr << "Usage: " << argv[0]
                      << " -base <base.fvecs> -graph <graph.bin> -out <codebook> [-seed <uint32>] [-device]\n";
            return 1;
        }
        const uint32_t seed = static_cast<uint32_t>(std::stoul(get(a, "-seed", "12345")));
        Buf v, e;
        uint64_t n = 0, ne = 0;
        uint32_t dim = 0, degree = 0;
        if (bs_read_graph(graph.c_str(), reinterpret_cast<uint32_t**>(&e.p), &ne, &degree))
            throw std::runtime_error(bs_host_last_error());
        if (bs_read_vecs(base.c_str(), 0, &v.p, &n, &dim)) throw std::runtime_error(bs_host_last_error());
        if (n != ne) throw std::runtime_error("graph and base sizes differ");
        const uint32_t pdim = bs_rabitq_padded_dim(dim), wpp = pdim / 32;
        std::cout << "dim=" << dim << " padded_dim=" << pdim << " degree=" << degree << " n=" << n
                  << " words_per_plane=" << wpp << "\n";
        std::vector<uint32_t> codes(n * degree * static_cast<uint64_t>(wpp));
        std::vector<float> factors(n * 3ull * degree), signs(pdim);
        uint32_t entry = 0;
        if (a.count("-device")) {
            bs_index ix = nullptr;
            if (bs_index_create(static_cast<float*>(v.p), static_cast<uint32_t*>(e.p), n, dim, degree, &ix) ||
                bs_index_build_rabitq(ix, seed, codes.data(), factors.data(), signs.data(), &entry)) {
                const std::string msg = bs_last_error();
                bs_index_destroy(ix);
                throw std::runtime_error(msg);
            }
            bs_index_destroy(ix);
        } else if (bs_build_rabitq(static_cast<float*>(v.p), static_cast<uint32_t*>(e.p), n, dim, degree, seed, 0,
                                   codes.data(), factors.data(), signs.data(), &entry)) {
            throw std::runtime_error(bs_host_last_error());
        }
        std::cout << "Entry point (medoid): " << entry << "\n";
        if (bs_write_codebook(out.c_str(), static_cast<float*>(v.p), static_cast<uint32_t*>(e.p), n, dim, degree, entry,
                              codes.data(), factors.data(), signs.data(), pdim))
            throw std::runtime_error(bs_host_last_error());
        std::cout << "Done. Codebook: " << out << "\n";
#elif BS_TOOL == 3
        auto a = args(argc, argv, {});
        const uint64_t n = std::stoull(get(a, "--n", "100000")), nq = std::stoull(get(a, "--nq", "1000"));
        const uint32_t dim = static_cast<uint32_t>(std::stoul(get(a, "--dim", "128")));
        const std::string kind = get(a, "--kind", "mixture");
        std::vector<float> b(n * dim), q(nq * dim);
        if (kind == "mixture") {
            const uint32_t c = static_cast<uint32_t>(std::stoul(get(a, "--centres", "64")));
            const float lo = std::stof(get(a, "--lo", "0")), hi = std::stof(get(a, "--hi", "128")),
                        sg = std::stof(get(a, "--sigma", "12"));
            bs_gen_mixture(b.data(), n, dim, c, lo, hi, sg, 0.0f, 101, 202);
            bs_gen_mixture(q.data(), nq, dim, c, lo, hi, sg, 0.0f, 101, 303);
        } else {
            bs_gen_normalized(b.data(), n, dim, 202);
            bs_gen_normalized(q.data(), nq, dim, 303);
        }
        if (bs_write_vecs(get(a, "--out-base", "base.fvecs").c_str(), 0, b.data(), n, dim) ||
            bs_write_vecs(get(a, "--out-query", "query.fvecs").c_str(), 0, q.data(), nq, dim))
            throw std::runtime_error(bs_host_last_error());
#elif BS_TOOL == 5
        if (argc != 5) {
            std::cerr << "Usage: replicate_queries <input.fvecs|ivecs> <output> <repeats> <format>\n"
                      << "  format: fvecs | ivecs\n";
            return 1;
        }
        const std::string fmt = argv[4];
        const long repeats = std::strtol(argv[3], nullptr, 10);
        if (repeats <= 0) {
            std::cerr << "repeats must be positive\n";
            return 1;
        }
        if (fmt != "fvecs" && fmt != "ivecs") {
            std::cerr << "Unknown format: " << fmt << " (use fvecs or ivecs)\n";
            return 1;
        }
        const int is_int = fmt == "ivecs";
        Buf in;
        uint64_t n = 0;
        uint32_t d = 0;
        if (bs_read_vecs(argv[1], is_int, &in.p, &n, &d)) throw std::runtime_error(bs_host_last_error());
        // both element types are 4 bytes: tile the raw rows
        const uint64_t row = static_cast<uint64_t>(d) * 4u, total = n * static_cast<uint64_t>(repeats);
        std::vector<unsigned char> out(total * row);
        for (long r = 0; r < repeats; ++r)
            if (n) std::memcpy(out.data() + static_cast<uint64_t>(r) * n * row, in.p, n * row);
        if (bs_write_vecs(argv[2], is_int, out.data(), total, d)) throw std::runtime_error(bs_host_last_error());
        std::cout << n << " x " << repeats << " = " << total << " vectors (dim=" << d << ") -> " << argv[2] << "\n";
#else
        auto a = args(argc, argv, {});
        Buf b, q;
        uint64_t n = 0, nq = 0;
        uint32_t d = 0, dq = 0;
        if (bs_read_vecs(get(a, "--base", "").c_str(), 0, &b.p, &n, &d) ||
            bs_read_vecs(get(a, "--query", "").c_str(), 0, &q.p, &nq, &dq))
            throw std::runtime_error(bs_host_last_error());
        const uint32_t k = static_cast<uint32_t>(std::stoul(get(a, "--k", "100")));
        std::vector<int32_t> gt(nq * k);
        bs_groundtruth(static_cast<float*>(b.p), n, static_cast<float*>(q.p), nq, d, k, gt.data(), 0);
        if (bs_write_vecs(get(a, "--out", "groundtruth.ivecs").c_str(), 1, gt.data(), nq, k))
            throw std::runtime_error(bs_host_last_error());
#endif
        return 0;
    } catch (const std::exception& e) {
        std::cerr << argv[0] << " error: " << e.what() << "\n";
        return 1;
    }
}
