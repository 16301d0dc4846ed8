// cli_config_check: gpu_cli's configuration reading (cli_config.hpp, json_lite.hpp) on one
// input, without touching any file or device, so that arbitrary and malformed configs can be
// run under the host sanitizers.  Reads the file named by argv[1] (stdin without one);
// prints "ok ..." and exits 0, or prints the CLI's error message and exits 1.
#include "cli_config.hpp"
#include "json_lite.hpp"

#include <fstream>
#include <iostream>
#include <iterator>
#include <sstream>
#include <string>

int main(int argc, char** argv) {
    std::string text;
    if (argc > 1) {
        std::ifstream f(argv[1], std::ios::binary);
        if (!f) {
            std::cerr << "cannot open " << argv[1] << std::endl;
            return 2;
        }
        text.assign((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    } else {
        text.assign((std::istreambuf_iterator<char>(std::cin)), std::istreambuf_iterator<char>());
    }
    jsonl::Value j;
    try {
        j = jsonl::parse(text);
    } catch (const std::exception& e) {
        std::cerr << "JSON parse error: " << e.what() << std::endl;
        return 1;
    }
    cli::DataFiles d;
    cli::SearchSettings s;
    std::string err = cli::read_data(j, d);
    if (err.empty()) err = cli::read_search_head(j, s);
    if (err.empty()) err = cli::read_search_rest(j, !d.codebook.empty(), s);
    if (!err.empty()) {
        std::cerr << err << std::endl;
        return 1;
    }
    std::cout << "ok mode=" << s.mode << " K=" << s.K << " topk_size=" << s.cfg.topk_size
              << " filter_capacity=" << s.cfg.filter_capacity << " max_iterations=" << s.cfg.max_iterations
              << " reset_interval=" << s.cfg.reset_interval << " queries_per_group=" << s.cfg.queries_per_group
              << " graph=" << d.graph << std::endl;
    return 0;
}
