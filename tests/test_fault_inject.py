"""Fault injection at the C ABI (nsmlp_fault_inject / NSMLP_FAULT_INJECT), on
the host: an armed entry point fails before it touches the device, with the
status and message a real failure of that kind gives, so a caller's failure
handling can be driven without a GPU fault.

The reference runtime tells an out-of-memory error by its message
(llama3_neuroplastic/experiments/runtime/_helpers.py:301-308); `_is_oom`
below restates that predicate so the test shows the injected message takes
the runtime's OOM branch (RT:5493-5524)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _is_oom(text: str) -> bool:
    t = text.lower()
    return ("out of memory" in t or "cudaerrormemoryallocation" in t or "cublas_status_alloc_failed" in t
            or "hip error out of memory" in t)


@pytest.fixture(scope="module")
def L():
    from next_step_ai_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from next_step_ai_amd import build_lib

        build_lib.build()
    lib = _lib.lib()
    yield lib
    _lib.fault_inject(None)


def _route(lib):
    # hidden size 100000 is rejected by validation when no fault fires
    return lib.nsmlp_route_f16(None, 1, 100000, None, None, 64, 64, None, None, None, 1664, 0, 208, None, None,
                               None, None, 0, None)


def test_disarmed_calls_validate_as_usual(L):
    from next_step_ai_amd import _lib

    _lib.fault_inject(None)
    assert _route(L) == -22 and b"hidden size" in L.nsmlp_last_error()


def test_count_limits_the_failing_calls(L):
    from next_step_ai_amd import _lib

    with _lib.injected_faults("route_f16=inval:2"):
        for _ in range(2):
            assert _route(L) == -22
            assert b"injected fault" in L.nsmlp_last_error() and b"nsmlp_route_f16" in L.nsmlp_last_error()
        assert _route(L) == -22 and b"hidden size" in L.nsmlp_last_error()  # the third call is a real one
    assert _route(L) == -22 and b"hidden size" in L.nsmlp_last_error()


@pytest.mark.parametrize("kind,code", [("hip", -5), ("inval", -22), ("nospc", -28), ("nodev", -19), ("oom", -5)])
def test_kinds_give_their_status(L, kind, code):
    from next_step_ai_amd import _lib

    with _lib.injected_faults(f"decode_layer_f16={kind}"):
        for _ in range(3):  # no count: every call
            rc = L.nsmlp_decode_layer_f16(None, None, None, 208, None, None, None, 0, None)
            assert rc == code
        msg = L.nsmlp_last_error().decode()
        assert _is_oom(msg) == (kind == "oom"), msg
        # other entry points are not armed
        assert _route(L) == -22 and b"hidden size" in L.nsmlp_last_error()


def test_wildcard_and_first_matching_rule(L):
    from next_step_ai_amd import _lib

    with _lib.injected_faults("route_f16=nodev:1,*=oom"):
        assert _route(L) == -19
        assert _route(L) == -5 and _is_oom(L.nsmlp_last_error().decode())  # rule 1 used up, the wildcard fires
        rc = L.nsmlp_single_kernel_decode_f16(None, None, None, None, None, None, None, None, None, None, None, None,
                                              16384, 32, 64, 208, None, 0, None)
        assert rc == -5
        # host-only calls are never armed
        assert L.nsmlp_version() >= 105
        assert L.nsmlp_decode_workspace_bytes(16384, 208) > 0


def test_python_call_raises_runtime_error_with_the_oom_message(L):
    from next_step_ai_amd import _lib

    with _lib.injected_faults("silu_mul_f16=oom"):
        with pytest.raises(RuntimeError) as ei:
            _lib.call("nsmlp_silu_mul_f16", None, None, None, 16, None)
    assert _is_oom(str(ei.value)), str(ei.value)


@pytest.mark.parametrize("spec", ["route_f16", "=hip", "route_f16=boom", "route_f16=hip:0", "route_f16=hip:x",
                                  "route_f16=hip:3:1", ",".join(["a=hip"] * 17)])
def test_bad_specs_are_refused_and_keep_the_rules(L, spec):
    from next_step_ai_amd import _lib

    with _lib.injected_faults("route_f16=nodev"):
        with pytest.raises(RuntimeError, match="bad fault-injection spec"):
            _lib.fault_inject(spec)
        assert _route(L) == -19  # the armed rule is still there


def _child(env_spec: str, body: str) -> str:
    env = dict(os.environ, NSMLP_FAULT_INJECT=env_spec)
    code = ("import sys; sys.path.insert(0, %r)\n" % ROOT) + "from next_step_ai_amd import _lib\nL = _lib.lib()\n" + body
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout


def test_environment_variable_arms_at_load():
    out = _child("route_f16=nodev:1", "print(L.nsmlp_route_f16(None, 1, 100000, None, None, 64, 64, None, None, None, "
                                      "1664, 0, 208, None, None, None, None, 0, None))\n"
                                      "print(L.nsmlp_route_f16(None, 1, 100000, None, None, 64, 64, None, None, None, "
                                      "1664, 0, 208, None, None, None, None, 0, None))\n")
    assert out.split() == ["-19", "-22"]


def test_bad_environment_spec_fails_every_compute_call():
    out = _child("route_f16=boom", "print(L.nsmlp_decode_layer_f16(None, None, None, 208, None, None, None, 0, None))\n"
                                   "print(L.nsmlp_last_error().decode())\n"
                                   "print(L.nsmlp_version())\n")
    lines = out.strip().splitlines()
    assert lines[0] == "-22" and "NSMLP_FAULT_INJECT" in lines[1] and int(lines[2]) >= 105
