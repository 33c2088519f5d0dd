// A GEMM problem in rocBLAS's column-major terms and the rocBLAS solution
// (Tensile kernel) chosen for it by measurement, for the table gemm_tuned.inc
// that blas.hip compiles in.
//
// The table is regenerated on an MI355X from a log of the problems the
// library itself issues (so that its keys match the calls exactly):
//   GPTC_GEMM_LOG=/tmp/gemms.txt python3 bench.py --workload gpt2 --steps 1 --warmup 0 --no-cpu-baseline
//   make -C gpt.c_amd tune && gpt.c_amd/_build/tune_gemm /tmp/gemms.txt > gpt.c_amd/csrc/gemm_tuned.inc
// tune_gemm (tune_gemm.cpp) times every solution rocBLAS lists for each
// problem of at least 1 GFLOP, re-times the fastest few, and keeps the winner
// only if it beats rocBLAS's default pick by 3 % or more, agrees with the
// default's result to 1e-5 of its largest entry and gives identical bits on
// a repeat.  Solution indices are those of this image's rocBLAS; another
// rocBLAS rejects them on first use and the default pick runs instead.
//
// Weight gradients: gptc_sgemm_wgrad uses the split count S of a tuned entry
// when the table has one for its product at S = 1, 2, 4 or 8 (one per
// product), else its tile-count rule.  Those entries come from a tune_gemm
// run over the four split counts of each product (log lines written by hand
// in the format above), the fastest GEMM plus its slices' add pass chosen.
#pragma once

namespace gptc {

struct GemmProblem {
    int ta, tb;              // op(A), op(B): 1 = transposed
    int m, n, k;             // C (m x n) = op(A) (m x k) op(B) (k x n), column-major
    int lda, ldb, ldc;
    long long sa, sb, sc;    // strides of a strided-batched problem (0 for a plain one)
    int batch;               // 0 for a plain GEMM
    int beta_zero, alpha_one;

    bool operator==(const GemmProblem &o) const {
        return ta == o.ta && tb == o.tb && m == o.m && n == o.n && k == o.k && lda == o.lda && ldb == o.ldb &&
               ldc == o.ldc && sa == o.sa && sb == o.sb && sc == o.sc && batch == o.batch &&
               beta_zero == o.beta_zero && alpha_one == o.alpha_one;
    }
};

struct GemmTuned {
    GemmProblem problem;
    int solution;
};

}  // namespace gptc
