"""The compiled-in table of rocBLAS solutions (gpt.c_amd/csrc/gemm_tuned.inc).

Each entry is a column-major rocBLAS problem and a solution index, matched
field for field against the library's calls (gpt.c_amd/csrc/blas.hip).
The table is data written by tune_gemm; these checks keep a hand edit or a
bad merge from naming a problem the library can never issue, two solutions
for one problem, or two split counts for one weight gradient (the library
takes the first it finds).  CPU only.
"""
import os
import re
from collections import Counter

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TABLE = os.path.join(ROOT, "gpt.c_amd", "csrc", "gemm_tuned.inc")
ENTRY = re.compile(r"^\{\{([-\d,\s]+)\},\s*(-?\d+)\},")


def entries():
    out = []
    for line in open(TABLE):
        line = line.strip()
        if not line or line.startswith("//"):
            continue
        m = ENTRY.match(line)
        assert m, f"unparsed table line: {line}"
        key = tuple(int(v) for v in m.group(1).split(","))
        assert len(key) == 14, line
        out.append((key, int(m.group(2))))
    return out


def test_table_entries_are_well_formed():
    es = entries()
    assert es, "the table is empty"
    for (ta, tb, m, n, k, lda, ldb, ldc, sa, sb, sc, batch, beta_zero, alpha_one), sol in es:
        assert ta in (0, 1) and tb in (0, 1) and beta_zero in (0, 1) and alpha_one in (0, 1)
        assert m > 0 and n > 0 and k > 0 and sol != 0
        assert lda >= (k if ta else m) and ldb >= (n if tb else k) and ldc >= m
        if batch == 0:
            assert sa == sb == sc == 0
        else:
            assert batch >= 2 and sa > 0 and sb > 0 and sc >= ldc * n


def test_table_keys_are_unique():
    keys = Counter(k for k, _ in entries())
    assert all(c == 1 for c in keys.values()), [k for k, c in keys.items() if c > 1]


def test_one_split_count_per_weight_gradient():
    """gptc_sgemm_wgrad's products: op(A) = N, op(B) = T, C = the (in x out)
    weight gradient, the reduction over rows cut into `batch` slices (or not,
    beta = 1 into dW).  One entry per product and total row count."""
    per_product = Counter()
    for (ta, tb, m, n, k, lda, ldb, ldc, sa, sb, sc, batch, beta_zero, _), _sol in entries():
        if ta == 0 and tb == 1:
            rows = k * (batch if batch else 1)
            if batch:
                assert beta_zero == 1 and sa == k * lda and sb == k * ldb and sc == m * n
            else:
                assert beta_zero == 0  # unsplit: accumulates into dW
            per_product[(m, n, rows)] += 1
    assert per_product and all(c == 1 for c in per_product.values()), per_product
