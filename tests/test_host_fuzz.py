"""Malformed inputs to the host parsers must be rejected without crashing: the JSON reader
behind sgl_qcfg_from_json and the safetensors reader (sgl_qst_open / get_raw).  Random and
mutated inputs, CPU only."""
import json
import random
import struct

import pytest

import sgl_qlinear as q

VALID_CFG = ('{"quantization_config": {"quant_method": "gptq", "bits": 4, "group_size": 128, '
             '"desc_act": false, "sym": true}}')


def _mutations(text, rng, n):
    b = bytearray(text.encode())
    for _ in range(n):
        c = bytearray(b)
        for _ in range(rng.randint(1, 6)):
            op = rng.randrange(4)
            i = rng.randrange(len(c)) if c else 0
            if op == 0 and c:
                c[i] = rng.randrange(256)
            elif op == 1 and c:
                del c[i:i + rng.randint(1, 8)]
            elif op == 2:
                c[i:i] = bytes(rng.randrange(256) for _ in range(rng.randint(1, 8)))
            else:
                c = c[:i]
        yield bytes(c)


def test_qcfg_json_fuzz():
    rng = random.Random(1)
    for s in _mutations(VALID_CFG, rng, 3000):
        q.qcfg_from_json(s.decode("latin-1"))  # any result; no crash
    deep = "[" * 100000 + "]" * 100000
    q.qcfg_from_json(deep)
    q.qcfg_from_json('{"quantization_config": ' + '{"a":' * 5000 + "1" + "}" * 5001)
    q.qcfg_from_json('{"quantization_config": {"bits": 1e999999, "group_size": -1e308}}')


def _st_bytes(header, data=b""):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


def test_safetensors_fuzz(tmp_path):
    rng = random.Random(2)
    good = {"w": {"dtype": "I32", "shape": [4, 4], "data_offsets": [0, 64]},
            "s": {"dtype": "F16", "shape": [2, 4], "data_offsets": [64, 80]}}
    base = json.dumps(good)
    p = tmp_path / "f.safetensors"
    for i, h in enumerate(_mutations(base, rng, 1500)):
        p.write_bytes(_st_bytes(h, bytes(80)))
        try:
            st = q.SafeTensors(p)
        except RuntimeError:
            continue
        for name in ("w", "s", "x", ""):
            st.get_raw(name)
        st.close()
    odd = [{"w": {"dtype": "I32", "shape": [4], "data_offsets": [64, 0]}},      # reversed
           {"w": {"dtype": "I32", "shape": [4], "data_offsets": [0, 10 ** 20]}},  # past end
           {"w": {"dtype": "I32", "shape": [], "data_offsets": [0, 0]}},
           {"w": {"dtype": "I32", "shape": [1, 2, 3, 4, 5], "data_offsets": [0, 4]}},
           {"w": {"dtype": 7, "shape": "x", "data_offsets": [0]}},
           {"w": {"dtype": "I32", "shape": [-3], "data_offsets": [-5, 4]}}]
    for h in odd:
        p.write_bytes(_st_bytes(h, bytes(80)))
        st = q.SafeTensors(p)
        r = st.get_raw("w")
        assert r is None or len(r[2]) <= 80
        st.close()
    for blob in (b"", b"\xff" * 7, struct.pack("<Q", 2 ** 63) + b"{}",
                 struct.pack("<Q", 3) + b"{}"):
        p.write_bytes(blob)
        with pytest.raises(RuntimeError):
            q.SafeTensors(p)


def test_probe_fuzzed_shapes(tmp_path):
    """Quantized-weight lookups over tensors with inconsistent shapes and dtypes never crash;
    probe reports -1 (error) or 0 (nothing there) or 1 with positive N, K."""
    rng = random.Random(3)
    p = tmp_path / "w.safetensors"
    dts = ["I32", "F16", "BF16", "F32", "U8", "I64", "F64"]
    for _ in range(400):
        names = [".qweight", ".qzeros", ".scales", ".g_idx", ".weight_packed", ".weight_scale",
                 ".weight_shape", ".weight"]
        hdr, off = {}, 0
        for n in rng.sample(names, rng.randint(1, len(names))):
            shape = [rng.choice([0, 1, 2, 3, 8, 16, 64, 128]) for _ in range(rng.randint(1, 3))]
            size = 1
            for d in shape:
                size *= d
            nb = size * rng.choice([1, 2, 4])
            hdr["b" + n] = {"dtype": rng.choice(dts), "shape": shape,
                            "data_offsets": [off, off + nb]}
            off += nb
        p.write_bytes(_st_bytes(hdr, bytes(off)))
        st = q.SafeTensors(p)
        for method in (1, 2, 3, 4):
            cfg = q.make_cfg(method=method, bits=rng.choice([4, 8]),
                             group_size=rng.choice([-1, 32, 128]), zero_point=rng.randint(0, 1),
                             layout=rng.randint(0, 1))
            rc, info = st.probe(cfg, "b")
            assert rc in (-1, 0, 1)
            if rc == 1:
                assert info["N"] > 0 and info["K"] > 0
        st.close()


def test_huge_dims_rejected(tmp_path):
    """Dimensions that do not fit (or are not whole numbers) make the tensor unreadable
    instead of overflowing the shape arithmetic."""
    p = tmp_path / "h.safetensors"
    for shape in ([1e30, 4], [2 ** 41, 1], [3.5, 2], [-1, 4]):
        h = {"b.qweight": {"dtype": "I32", "shape": shape, "data_offsets": [0, 16]},
             "b.scales": {"dtype": "F16", "shape": [1, 4], "data_offsets": [16, 24]}}
        p.write_bytes(_st_bytes(h, bytes(24)))
        st = q.SafeTensors(p)
        assert st.get_raw("b.qweight") is None
        assert st.probe(q.make_cfg(method=2, bits=4, group_size=128), "b")[0] == 0
        st.close()
