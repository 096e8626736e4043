"""mlamoe.weights -- the offline int8 expert format ("mlamoe-i8") and its
loader.

The reference keeps its experts as bf16 safetensors tensors and packs them
for its kernels at start-up (src/getp_run.hip:58-113, 797-808).  The int8
MFMA kernels of this library read a per-layer pool of 16-row x 64-byte
fragments with one fp32 scale per output row (include/mlamoe.h, "the packed
int8 expert format").  This module

  * quantises and packs bf16 expert weights on the host, bit-identical to the
    device path of mm_moe_load_layer(MM_LOAD_INT8) (mm_quant_weight +
    mm_pack_i8);
  * reads a checkpoint laid out as the reference loads it (model.safetensors
    or model.safetensors.index.json; tensor names of src/model_load.c:118-148);
  * writes / reads the packed layers as a safetensors container (header
    metadata "format": "mlamoe-i8");
  * uploads packed layers with mm_moe_load_layer_i8_packed (no quantisation
    at load).

safetensors container (public format): an 8-byte little-endian header
length, a JSON header {name: {dtype, shape, data_offsets}, "__metadata__":
{str: str}}, then the data.  bf16 tensors are handled as uint16.
"""
from __future__ import annotations

import ctypes as C
import json
import mmap
import os
import struct

import numpy as np

FORMAT = "mlamoe-i8"
VERSION = "1"

_NP = {"BF16": np.uint16, "F32": np.float32, "I8": np.int8, "U8": np.uint8, "F16": np.float16,
       "I32": np.int32, "I64": np.int64, "U16": np.uint16}


# ---- safetensors container ---------------------------------------------------

class SafeTensors:
    """Memory-mapped read-only view of one .safetensors file."""

    def __init__(self, path):
        self.path = path
        with open(path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        (n,) = struct.unpack("<Q", self._mm[:8])
        hdr = json.loads(self._mm[8:8 + n].decode("utf-8"))
        self.metadata = hdr.pop("__metadata__", {}) or {}
        self._hdr = hdr
        self._base = 8 + n

    def names(self):
        return list(self._hdr)

    def dtype(self, name):
        return self._hdr[name]["dtype"]

    def get(self, name):
        h = self._hdr[name]
        if h["dtype"] not in _NP:
            raise ValueError(f"{self.path}: {name}: dtype {h['dtype']} not supported")
        b0, b1 = h["data_offsets"]
        a = np.frombuffer(self._mm, dtype=_NP[h["dtype"]], count=(b1 - b0) // np.dtype(_NP[h["dtype"]]).itemsize,
                          offset=self._base + b0)
        return a.reshape(h["shape"])


def write_safetensors(path, tensors, metadata=None):
    """tensors: {name: (dtype string, numpy array)} written in insertion
    order, each 8-byte aligned."""
    hdr, off, blobs = {}, 0, []
    for name, (dt, a) in tensors.items():
        a = np.ascontiguousarray(a, dtype=_NP[dt])
        pad = (-off) % 8
        if pad:
            blobs.append(b"\0" * pad)
            off += pad
        hdr[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + a.nbytes]}
        blobs.append(a.tobytes())
        off += a.nbytes
    if metadata:
        hdr["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    h = json.dumps(hdr, separators=(",", ":")).encode("utf-8")
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


class Checkpoint:
    """The tensors of a model directory as the reference opens it:
    model.safetensors.index.json's weight_map over its shards, or a single
    model.safetensors."""

    def __init__(self, model_dir):
        self.dir = model_dir
        idx = os.path.join(model_dir, "model.safetensors.index.json")
        self._files, self._where = {}, {}
        if os.path.exists(idx):
            wm = json.load(open(idx))["weight_map"]
            for name, shard in wm.items():
                self._where[name] = shard
        else:
            st = self._file("model.safetensors")
            for name in st.names():
                self._where[name] = "model.safetensors"
        cfg = os.path.join(model_dir, "config.json")
        self.config = json.load(open(cfg)) if os.path.exists(cfg) else {}

    def _file(self, shard):
        if shard not in self._files:
            self._files[shard] = SafeTensors(os.path.join(self.dir, shard))
        return self._files[shard]

    def has(self, name):
        return name in self._where

    def get(self, name):
        if name not in self._where:
            raise KeyError(f"{self.dir}: tensor {name} not found")
        return self._file(self._where[name]).get(name)


# ---- quantisation and fragment packing ----------------------------------------

def quantize_rows(w):
    """Per-row int8 quantisation of bf16 rows (uint16 [..., N, K]): s =
    max|w| / 127 in fp32, q = clamp(rint(w / s), -127, 127), q = 0 where s == 0
    -- the device's mm_quant_weight step for step."""
    w = np.ascontiguousarray(w, np.uint16)
    f = (w.astype(np.uint32) << 16).view(np.float32)
    amax = np.abs(f).max(axis=-1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(s == 0, np.float32(1.0), s).astype(np.float32)
    q = np.clip(np.rint(f / safe[..., None]), -127, 127)
    q[s == 0] = 0
    return q.astype(np.int8), s


def pack(q0, q1=None):
    """Fragments of int8 rows q [..., N, K] (N % 16 == 0, K % 64 == 0): for
    row block nb and 64-byte column block kb, fragment byte 16 l + b holds
    row 16 nb + (l % 16), column 64 kb + 16 (l / 16) + b; with q1 the two
    matrices' fragments alternate (gate, up).  Returns int8 [..., N*K*(1|2)]."""
    N, K = q0.shape[-2:]
    lead = q0.shape[:-2]
    parts = []
    for q in (q0,) if q1 is None else (q0, q1):
        q = np.ascontiguousarray(q, np.int8).reshape(*lead, N // 16, 16, K // 64, 4, 16)
        n = len(lead)
        parts.append(q.transpose(*range(n), n, n + 2, n + 3, n + 1, n + 4))
    out = parts[0][..., None, :, :, :] if q1 is None else np.stack(parts, axis=len(lead) + 2)
    return np.ascontiguousarray(out).reshape(*lead, -1)


def unpack(buf, N, K, two=False):
    """Inverse of pack for one matrix (or a gate/up pair)."""
    ns = 2 if two else 1
    a = np.asarray(buf, np.int8).reshape(N // 16, K // 64, ns, 4, 16, 16)
    qs = [a[:, :, i].transpose(0, 3, 1, 2, 4).reshape(N, K) for i in range(ns)]
    return tuple(qs) if two else qs[0]


def layer_sizes(H, E, I, n_shared):
    """(pool bytes, scale count) of one packed layer (mm_moe_i8_layer_size)."""
    S = n_shared * I
    return 3 * E * I * H + 3 * S * H, 2 * E * I + E * H + 2 * S + H


def pack_layer(w, H, E, I, n_shared):
    """One MoE layer's bf16 experts (dict as mlamoe.synth.moe_layer: eg/eu
    [E, I, H], ed [E, H, I], sg/su [S, H], sd [H, S]) -> (pool int8, scales
    fp32) in the device layout."""
    S = n_shared * I
    qg, sg = quantize_rows(np.asarray(w["eg"]).reshape(E, I, H))
    qu, su = quantize_rows(np.asarray(w["eu"]).reshape(E, I, H))
    qd, sd = quantize_rows(np.asarray(w["ed"]).reshape(E, H, I))
    pool = [pack(qg, qu).reshape(-1), pack(qd).reshape(-1)]
    scales = [sg.reshape(-1), su.reshape(-1), sd.reshape(-1)]
    if S:
        qsg, ssg = quantize_rows(np.asarray(w["sg"]).reshape(S, H))
        qsu, ssu = quantize_rows(np.asarray(w["su"]).reshape(S, H))
        qsd, ssd = quantize_rows(np.asarray(w["sd"]).reshape(H, S))
        pool += [pack(qsg, qsu), pack(qsd)]
        scales += [ssg, ssu]
    else:
        ssd = np.zeros(H, np.float32)
    scales.append(ssd)
    pool, scales = np.concatenate(pool), np.concatenate(scales).astype(np.float32)
    assert (pool.size, scales.size) == layer_sizes(H, E, I, n_shared)
    return pool, scales


# ---- checkpoints -> packed file -------------------------------------------------

def moe_layer_from_checkpoint(ck, layer, E):
    """One MoE layer's weights by the reference's tensor names
    (src/model_load.c:118-148), experts stacked."""
    p = f"model.layers.{layer}.mlp"
    w = dict(moe_gate=ck.get(f"{p}.gate.weight"),
             moe_gate_bias=ck.get(f"{p}.gate.e_score_correction_bias")
             if ck.has(f"{p}.gate.e_score_correction_bias") else None,
             sg=ck.get(f"{p}.shared_experts.gate_proj.weight"),
             su=ck.get(f"{p}.shared_experts.up_proj.weight"),
             sd=ck.get(f"{p}.shared_experts.down_proj.weight"))
    for key, proj in (("eg", "gate_proj"), ("eu", "up_proj"), ("ed", "down_proj")):
        w[key] = np.stack([ck.get(f"{p}.experts.{e}.{proj}.weight") for e in range(E)])
    return w


def _geometry(cfg):
    return (int(cfg["hidden_size"]), int(cfg["n_routed_experts"]),
            int(cfg["moe_intermediate_size"]), int(cfg.get("n_shared_experts", 0) or 0))


def convert(model_dir, out_path, layers=None):
    """Quantise and pack every MoE layer of a checkpoint (layers
    first_k_dense_replace .. num_hidden_layers - 1 by default) into one
    mlamoe-i8 file.  Returns the list of layers written."""
    ck = Checkpoint(model_dir)
    cfg = ck.config
    H, E, I, NS = _geometry(cfg)
    if layers is None:
        layers = list(range(int(cfg.get("first_k_dense_replace", 0)), int(cfg["num_hidden_layers"])))
    tensors = {}
    for l in layers:
        w = moe_layer_from_checkpoint(ck, l, E)
        pool, scales = pack_layer(w, H, E, I, NS)
        p = f"model.layers.{l}.mlp"
        tensors[f"{p}.experts.i8_pool"] = ("I8", pool)
        tensors[f"{p}.experts.i8_scales"] = ("F32", scales)
        tensors[f"{p}.gate.weight"] = ("BF16", np.asarray(w["moe_gate"], np.uint16))
        if w["moe_gate_bias"] is not None:
            tensors[f"{p}.gate.e_score_correction_bias"] = ("F32", np.asarray(w["moe_gate_bias"]))
    write_safetensors(out_path, tensors, dict(
        format=FORMAT, version=VERSION, hidden_size=H, n_routed_experts=E,
        moe_intermediate_size=I, n_shared_experts=NS, layers=",".join(map(str, layers))))
    return layers


def save_packed(out_path, H, E, I, n_shared, layers):
    """layers: {l: (pool, scales, moe_gate, moe_gate_bias or None)}."""
    tensors = {}
    for l, (pool, scales, gate, bias) in layers.items():
        p = f"model.layers.{l}.mlp"
        tensors[f"{p}.experts.i8_pool"] = ("I8", pool)
        tensors[f"{p}.experts.i8_scales"] = ("F32", scales)
        tensors[f"{p}.gate.weight"] = ("BF16", gate)
        if bias is not None:
            tensors[f"{p}.gate.e_score_correction_bias"] = ("F32", bias)
    write_safetensors(out_path, tensors, dict(
        format=FORMAT, version=VERSION, hidden_size=H, n_routed_experts=E,
        moe_intermediate_size=I, n_shared_experts=n_shared, layers=",".join(map(str, layers))))


def read_packed(path):
    """(geometry dict, reader, layer list) of an mlamoe-i8 file; raises on
    another format or version."""
    st = SafeTensors(path)
    m = st.metadata
    if m.get("format") != FORMAT or m.get("version") != VERSION:
        raise ValueError(f"{path}: not an {FORMAT} v{VERSION} file (metadata {m})")
    geo = {k: int(m[k]) for k in ("hidden_size", "n_routed_experts", "moe_intermediate_size",
                                  "n_shared_experts")}
    layers = [int(v) for v in m["layers"].split(",") if v != ""]
    return geo, st, layers


def load(ctx, path, layer_map=None):
    """Upload every layer of an mlamoe-i8 file into ctx (mm_moe_init done
    with the same geometry) through mm_moe_load_layer_i8_packed.
    layer_map: {file layer: context layer}, default identity."""
    from . import _check, lib
    geo, st, layers = read_packed(path)
    cfg = ctx._moe_cfg
    got = (cfg.hidden_size, cfg.n_routed_experts, cfg.moe_inter_size, cfg.n_shared_experts)
    want = (geo["hidden_size"], geo["n_routed_experts"], geo["moe_intermediate_size"],
            geo["n_shared_experts"])
    if got != want:
        raise ValueError(f"{path}: geometry {want} does not match the context's {got}")
    for l in layers:
        p = f"model.layers.{l}.mlp"
        pool = np.ascontiguousarray(st.get(f"{p}.experts.i8_pool"))
        scales = np.ascontiguousarray(st.get(f"{p}.experts.i8_scales"))
        gate = np.ascontiguousarray(st.get(f"{p}.gate.weight"))
        bn = f"{p}.gate.e_score_correction_bias"
        bias = np.ascontiguousarray(st.get(bn)) if bn in st.names() else None
        _check(lib().mm_moe_load_layer_i8_packed(
            ctx.h, (layer_map or {}).get(l, l), gate.ctypes.data,
            bias.ctypes.data if bias is not None else None, pool.ctypes.data,
            scales.ctypes.data, 0))
    return layers


def layer_size(cfg):
    """(pool bytes, scale count) from the library (mm_moe_i8_layer_size)."""
    from . import _check, lib
    pb, ns = C.c_size_t(), C.c_size_t()
    _check(lib().mm_moe_i8_layer_size(C.byref(cfg), C.byref(pb), C.byref(ns)))
    return pb.value, ns.value
