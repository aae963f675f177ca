"""CPU-side tests of the drop-in boundary: the C ABI library, the pybind11 module and the
Python shim's checks.  No kernel is launched: every call here returns before any HIP call
(argument validation happens first, include/tfgfa.h)."""
import ctypes
import os
import re
import types

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tfgfa.h")

import custom_flash_attn  # noqa: E402
from custom_flash_attn import _C  # noqa: E402


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tfgfa_\w+)\s*\(", text)))


def _header_define(name):
    m = re.search(rf"#define\s+{name}\s+(-?\d+)", open(HEADER).read())
    return int(m.group(1))


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(custom_flash_attn.library_path())
    lib.tfgfa_fwd_bf16.restype = ctypes.c_int
    lib.tfgfa_fwd_bf16.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_void_p] + [ctypes.c_int] * 4 + [
        ctypes.c_float, ctypes.c_int, ctypes.c_void_p]
    lib.tfgfa_strerror.restype = ctypes.c_char_p
    lib.tfgfa_strerror.argtypes = [ctypes.c_int]
    lib.tfgfa_abi_version.restype = ctypes.c_int
    return lib


def test_library_exports_every_declared_symbol(lib):
    names = _header_functions()
    assert names == ["tfgfa_abi_version", "tfgfa_device_info", "tfgfa_fwd_bf16", "tfgfa_strerror"]
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/tfgfa.h but not exported"


def test_abi_version(lib):
    assert lib.tfgfa_abi_version() == _header_define("TFGFA_ABI_VERSION")
    assert _C.abi_version() == _header_define("TFGFA_ABI_VERSION")


def test_strerror_covers_every_status(lib):
    codes = [_header_define(n) for n in (
        "TFGFA_OK", "TFGFA_ERR_NULL_POINTER", "TFGFA_ERR_BAD_SHAPE", "TFGFA_ERR_HEAD_DIM",
        "TFGFA_ERR_SCALE", "TFGFA_ERR_CAUSAL_FLAG", "TFGFA_ERR_TOO_LARGE", "TFGFA_ERR_ALIGNMENT")]
    msgs = [lib.tfgfa_strerror(c).decode() for c in codes]
    assert len(set(msgs)) == len(msgs)
    assert lib.tfgfa_strerror(12345).decode() == "unknown tfgfa status"
    assert _C.strerror(3) == msgs[3]


# Fake, 16-byte-aligned device addresses: validation never dereferences them.
P = 0x10000


@pytest.mark.parametrize("args,code", [
    ((0, P, P, P, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_NULL_POINTER"),
    ((P, P, P, 0, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_NULL_POINTER"),
    ((P, P, P, P, 0, -1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_BAD_SHAPE"),
    ((P, P, P, P, 0, 1, 1, -16, 64, 0.125, 1), "TFGFA_ERR_BAD_SHAPE"),
    ((P, P, P, P, 0, 1, 1, 16, 128, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),
    ((P, P, P, P, 0, 1, 1, 16, 32, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),
    ((P, P, P, P, 0, 1, 1, 16, 64, 0.0, 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, -0.125, 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, float("nan"), 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, float("inf"), 1), "TFGFA_ERR_SCALE"),
    ((P, P, P, P, 0, 1, 1, 16, 64, 0.125, 2), "TFGFA_ERR_CAUSAL_FLAG"),
    ((P + 2, P, P, P, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_ALIGNMENT"),
    ((P, P, P, P + 8, 0, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_ALIGNMENT"),
    ((P, P, P, P, P + 2, 1, 1, 16, 64, 0.125, 1), "TFGFA_ERR_ALIGNMENT"),
    ((P, P, P, P, 0, 65536, 65536, 16, 64, 0.125, 1), "TFGFA_ERR_TOO_LARGE"),
    ((P, P, P, P, 0, 1, 1, 1 << 30, 64, 0.125, 1), "TFGFA_ERR_TOO_LARGE"),
    ((P, P, P, P, 0, 0, 4, 16, 64, 0.125, 1), "TFGFA_OK"),   # empty problem: nothing launched
    ((P, P, P, P, 0, 2, 4, 0, 64, 0.125, 0), "TFGFA_OK"),
    ((0, 0, 0, 0, 0, 2, 4, 0, 64, 0.125, 1), "TFGFA_OK"),     # empty tensors have NULL data
    ((0, 0, 0, 0, 0, 2, 4, 0, 128, 0.125, 1), "TFGFA_ERR_HEAD_DIM"),  # sizes checked first
])
def test_c_abi_argument_validation(lib, args, code):
    assert lib.tfgfa_fwd_bf16(*args, None) == _header_define(code)


def test_pybind_raises_runtime_error_with_message():
    with pytest.raises(RuntimeError, match="unsupported head dimension"):
        _C.fwd(P, P, P, P, 0, 1, 1, 16, 128, 0.125, True, 0)
    with pytest.raises(RuntimeError, match="null tensor pointer"):
        _C.fwd(0, P, P, P, 0, 1, 1, 16, 64, 0.125, True, 0)


# ------------------------------------------------------------------ shim checks


def test_forward_rejects_cpu_tensors_like_the_reference():
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="^Q must be a CUDA tensor$"):
        custom_flash_attn.forward(q, q, q)
    with pytest.raises(RuntimeError, match="^Q must be a CUDA tensor$"):
        custom_flash_attn.forward_lse(q, q, q)


class _FakeCuda:
    """Stands in for a device tensor so the shim's later checks can run on the CPU."""

    def __init__(self, shape=(1, 2, 8, 64), dtype=torch.bfloat16, contiguous=True, device="cuda:0"):
        self.shape = torch.Size(shape)
        self.dtype = dtype
        self.is_cuda = True
        self._contig = contiguous
        self.device = torch.device(device)

    def is_contiguous(self):
        return self._contig

    def dim(self):
        return len(self.shape)


@pytest.mark.parametrize("qkv,msg", [
    ((_FakeCuda(contiguous=False), _FakeCuda(), _FakeCuda()), "^Q must be contiguous$"),
    ((_FakeCuda(), _FakeCuda(contiguous=False), _FakeCuda()), "^K_mat must be contiguous$"),
    ((_FakeCuda(), _FakeCuda(), _FakeCuda(contiguous=False)), "^V must be contiguous$"),
    ((_FakeCuda(dtype=torch.float16),) * 3, r"^Unsupported tensor dtype. Use bfloat16.$"),
    ((_FakeCuda(dtype=torch.float32),) * 3, r"^Unsupported tensor dtype. Use bfloat16.$"),
    ((_FakeCuda(), _FakeCuda(dtype=torch.float16), _FakeCuda()), r"^Unsupported tensor dtype"),
    ((_FakeCuda(shape=(2, 8, 64)),) * 3, "must be 4-D"),
    ((_FakeCuda(), _FakeCuda(shape=(1, 2, 9, 64)), _FakeCuda()), "same shape"),
    ((_FakeCuda(), _FakeCuda(), _FakeCuda(device="cuda:1")), "same device"),
    ((_FakeCuda(shape=(1, 2, 8, 128)),) * 3, "head_dim must be 64"),
])
def test_shim_validation_messages(qkv, msg):
    with pytest.raises(RuntimeError, match=msg):
        custom_flash_attn._validate(*qkv)


def test_forward_is_positional_only():
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        custom_flash_attn.forward(Q=q, K_mat=q, V=q)


# ------------------------------------------------------------------ GPT-2 caller (CPU)


def test_gpt2_manual_and_functional_agree_on_cpu():
    import model_inference as mi

    cfg = dict(mi.GPT_CONFIG_124M)
    cfg.update({"emb_dim": 128, "n_layers": 2, "n_heads": 2, "vocab_size": 97,
                "context_length": 64, "drop_rate": 0.0, "qkv_bias": True})
    outs = {}
    for impl in ("manual", "functional"):
        torch.manual_seed(0)
        model = mi.GPTModel(dict(cfg, impl_type=impl)).eval()
        mi.init_gpt2_weights(model, seed=7)
        idx = torch.randint(0, 97, (2, 40), generator=torch.Generator().manual_seed(3))
        with torch.no_grad():
            outs[impl] = model(idx)
    assert outs["manual"].shape == (2, 40, 97)
    torch.testing.assert_close(outs["manual"], outs["functional"], rtol=1e-4, atol=1e-5)


def test_gpt2_rejects_unknown_impl():
    import model_inference as mi

    with pytest.raises(ValueError, match="triton"):
        mi.MultiHeadAttention(8, 8, 4, 0.0, 2, "triton")
