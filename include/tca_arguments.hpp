// tca_arguments.hpp -- the Arguments class: command-line flags of the ./test
// harness, and the options the reference-signature readers of tca_compat.hpp
// take (mtx_input_to_CSR, mtx_input_to_Dense, smtx_input_to_CSR read
// pattern_only and input_is_zero_based).
//
// Same getopt letters, defaults and meanings as the reference's Arguments
// class (src/arg_parse.h:15-161), which its main() never instantiated; here
// main() honours them.  Differences, all deliberate:
//   * N defaults to 256 when a matrix file is given (the reference harness
//     hard-codes N = 256, src/test.cu:47); the Arguments default 1024 applies
//     to synthetic matrices;
//   * -d 1 selects fp32 A/B (the reference rejects it as not implemented);
//     -d 3 selects bf16; -d 2 (fp64) is rejected: there is no fp64 path;
//   * the matrix file may also be given as the first positional argument
//     (the reference's "./test {matrix.smtx}" usage, src/test.cu:38-43);
//   * -f stores the full name (the reference under-allocates by one byte,
//     src/arg_parse.h:79) in a std::string; -r sets the seed of B; -j prints
//     a JSON summary;
//   * the constructor does not print; print() gives the reference's summary;
//   * a default-constructed Arguments holds the defaults (for callers of the
//     readers that build their options in code).
#pragma once

#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <string>

#include "tca_spmm.h"

class Arguments {
  public:
    int M = 1024;
    int N = 1024;
    int K = 1024;
    int num_iter = 10;
    bool pattern_only = false;
    bool input_is_zero_based = true;
    bool input_file_exists = false;
    float target_sparsity = 0.8f;
    float tolerance = 1e-3f;
    int dtype = TCA_F16;  // A and B; C is fp32
    std::string input_fname;
    int ell_block_size = 32;  // -e: Blocked-ELL block size (printed; the harness runs the CSR SpMM,
                              // the Blocked-ELL kernel is tca_bell_spmm / bench.py --bell)
    unsigned long long seed = 1;
    bool json = false;
    bool n_given = false;

    Arguments() = default;
    Arguments(int argc, char* argv[]) { ParseArgs(argc, argv); }

    // The reference's summary of the options (src/arg_parse.h:130-158).
    void print() const {
        static const char* names[] = {"FP16", "FP32", "BF16"};
        const char* ab = names[dtype == TCA_F32 ? 1 : dtype == TCA_BF16 ? 2 : 0];
        std::printf("===================== Arguments ==========================\n");
        std::printf("Tolerance : %f\n", tolerance);
        std::printf("A type : %s, B type : %s, C type : %s\n", ab, ab, "FP32");
        std::printf("N iter : %d\n", num_iter);
        std::printf("Ell block size : %d \n", ell_block_size);
        if (!input_file_exists) {
            std::printf("No input file have been passed ... generate synthetic with random entries\n");
            std::printf("The matrix size .. M: %d , N: %d, K: %d\n", M, N, K);
            std::printf("Target Sparsity : %f\n", target_sparsity);
        } else {
            std::printf("Input file name : %s\n", input_fname.c_str());
            if (pattern_only) std::printf("Matrix is specified as pattern only matrix\n");
            if (!input_is_zero_based) std::printf("Input matrix is specified as one based index matrix\n");
        }
        std::printf("================== End of Arguments ======================\n");
    }

    static void usage(const char* prog) {
        std::printf(
            "Usage : %s [options] {matrix.smtx | matrix.mtx}\n"
            "  -f file   input matrix (.smtx, or .mtx MatrixMarket coordinate)\n"
            "  -n N      dense width of B and C (default 256 with a file, else 1024)\n"
            "  -m M -k K -s sparsity   synthetic A when no file is given (defaults 1024, 1024, 0.8)\n"
            "  -i iters  timed launches (default 10, after 5 warm-ups)\n"
            "  -t tol    validation tolerance (default 1e-3)\n"
            "  -d type   0: fp16 A/B (default), 1: fp32, 3: bf16; C is fp32 (2: fp64 not implemented)\n"
            "  -p 0|1    .mtx pattern only;  -b 0|1  .mtx zero (0) or one (1) based\n"
            "  -e size   ell block size (accepted, unused)\n"
            "  -r seed   seed of B;  -j  print a JSON summary line\n",
            prog);
    }

    void ParseArgs(int argc, char* argv[]) {
        int c;
        while ((c = getopt(argc, argv, "m:n:k:i:t:s:f:d:p:b:e:r:jh")) != -1) {
            switch (c) {
                case 'm': M = std::stoi(optarg); break;
                case 'n': N = std::stoi(optarg); n_given = true; break;
                case 'k': K = std::stoi(optarg); break;
                case 'i': num_iter = std::stoi(optarg); break;
                case 't': tolerance = std::stof(optarg); break;
                case 's': target_sparsity = std::stof(optarg); break;
                case 'f': input_fname = optarg; break;
                case 'p': pattern_only = std::stoi(optarg) == 1; break;
                case 'b': input_is_zero_based = std::stoi(optarg) == 0; break;
                case 'e': ell_block_size = std::stoi(optarg); break;
                case 'r': seed = std::stoull(optarg); break;
                case 'j': json = true; break;
                case 'd': {
                    const int d = std::stoi(optarg);
                    if (d == 0) dtype = TCA_F16;
                    else if (d == 1) dtype = TCA_F32;
                    else if (d == 3) dtype = TCA_BF16;
                    else {
                        std::fprintf(stderr, "Not Implemented error for the specified dtype\n");
                        std::exit(EXIT_FAILURE);
                    }
                    break;
                }
                case 'h': usage(argv[0]); std::exit(EXIT_SUCCESS);
                default: usage(argv[0]); std::exit(EXIT_FAILURE);
            }
        }
        if (input_fname.empty() && optind < argc) input_fname = argv[optind];
        if (!input_fname.empty() && access(input_fname.c_str(), F_OK) != 0) {
            std::fprintf(stderr, "Input file not exists error\n");
            std::exit(EXIT_FAILURE);
        }
        input_file_exists = !input_fname.empty();
        if (input_file_exists && !n_given) N = 256;
        if (N < 1 || M < 0 || K < 1 || num_iter < 1) {
            std::fprintf(stderr, "invalid sizes\n");
            std::exit(EXIT_FAILURE);
        }
    }
};
