import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "talos-xii_amd"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP path through the C ABI")


@pytest.fixture(scope="session")
def oracle():
    import pyoracle
    # the prebuilt checker (__graft_entry__.build() compiles it before any test runs; building it
    # here could start the compiler from a process that has already initialised the GPU)
    pyoracle.lib()
    # the CPU share of a GPU box is 16 cores whatever the machine reports
    pyoracle.set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    return pyoracle


def pytest_terminal_summary(terminalreporter):
    """The parameter-gradient tolerance audit: every tensor with elements that needed the
    magnitude-derived allowance (common.check_grad) to pass, how many, and the kappa they needed."""
    try:
        import common
    except ImportError:
        return
    recs = common.GRAD_AUDIT
    if not recs:
        return
    out = os.environ.get("TALOS_TOLERANCE_AUDIT")
    if out:
        with open(out, "w") as f:
            json.dump(recs, f, indent=1)
    tr = terminalreporter
    tr.section("parameter-gradient tolerance audit")
    for rule, plain, unit in (("fp32", "1e-4 |ref| + 1e-5", "2^-24"), ("bf16", "2e-2 |ref| + 1e-5", "2^-8")):
        rs = [r for r in recs if r.get("rule", "fp32") == rule]
        if not rs:
            continue
        need = [r for r in rs if r["needs_mag"]]
        worst = max(r["kappa_needed"] for r in rs)
        tr.write_line(f"{rule}: {len(rs)} parameter-gradient tensors checked; {len(need)} have elements beyond the "
                      f"plain {plain} rule; largest kappa needed {worst:.2f} (allowed {rs[0]['kappa']:.0f}, "
                      f"unit {unit})")
        for r in sorted(need, key=lambda r: -r["kappa_needed"]):
            tr.write_line(f"  {r['test']} {r['tensor']}: {r['needs_mag']}/{r['size']} elements beyond the plain "
                          f"rule, kappa needed {r['kappa_needed']:.2f}, worst err / plain bound "
                          f"{r['worst_err_over_plain']:.2f} (max|ref| {r['max_abs_ref']:.3e})")
