"""Reader for FreeML model checkpoints (the files ``Model::Save`` writes) and the NanoLLM
parameter set they hold.

On-disk layout, as written by Model::Save (ModelLibrary/Model.h:91-159) through SaveLoader
(Loading/SaveLoader.h):

* ``<dir>/model.guide`` (Model.h:343-379): one ``LAYER <guid> <file>`` line per layer in
  ``m_allLayers`` order, then ``INPUT_DIMS x y z``, ``OPTIMISER <file|0> 0``,
  ``LOSSFUNC <file|0> 0``.  ``<dir>`` is ``<cwd>/<sanitised model name>`` (Model.h:94).
* ``*.blob_layer`` (SaveLoader.h:499-583, parsed as in :676-781): text records of
  ``NAME`` / ``DATA`` / ``TYPE`` [/ ``META`` / ``GUID``] lines closed by ``;``.  The record
  named ``Layer_Name`` carries the layer's name (DATA), ``ROOTLAYER_<type>`` and its GUID;
  ``LAYER_<type>`` records point at a sub-layer's own ``.blob_layer``; ``INT`` / ``UINT`` /
  ``FLOAT`` records at a ``.blob_data`` file holding one 4-byte value; ``MATRIX`` records at a
  ``.blob_matrix`` file.
* ``*.blob_matrix`` (SaveLoader.h:1523-1545, parsed as in :1267-1348): ``INTERNAL_NAME``,
  ``GUID``, ``DIMX``, ``DIMY``, ``DIMZ``, ``DATA <file>``; the data file is the matrix's
  ``GetRawData`` bytes, DIMX*DIMY*DIMZ float32 with x fastest.  Two matrices with one GUID
  are one matrix (SaveLoader.h:1358-1364): this is how a tied lm_head is stored.

``load_nanollm(dir)`` turns a checkpoint of the NanoLLM graph (Examples/NanoLLM/NanoLLM.cpp:
255-376) into ``synth.NanoLLMWeights``, which ``freeml_amd.NanoLLM`` uploads.  The reader is
host-side file parsing only; nothing here computes on the model.
"""
from __future__ import annotations

import dataclasses
import os

import numpy as np

from .synth import LayerWeights, NanoLLMShape, NanoLLMWeights


class CheckpointError(ValueError):
    """The directory is not a readable FreeML checkpoint of the expected graph."""


@dataclasses.dataclass
class MatrixRecord:
    """One ``.blob_matrix`` entry; ``array()`` reads its data file as (DIMZ, DIMY, DIMX)."""

    path: str
    name: str
    guid: int | None
    dims: tuple  # (x, y, z)
    data_file: str

    def array(self) -> np.ndarray:
        x, y, z = self.dims
        n = x * y * z
        raw = np.fromfile(self.data_file, dtype="<f4")
        if raw.size != n:
            raise CheckpointError(f"{self.path}: {raw.size} floats in {self.data_file}, dims "
                                  f"{x}x{y}x{z} need {n}")
        return raw.reshape(z, y, x)


@dataclasses.dataclass
class LayerRecord:
    """One ``.blob_layer`` file: a layer (or sub-layer blob) with its values and matrices."""

    path: str
    name: str = ""
    type: str = ""
    meta: str = ""
    guid: int | None = None
    sublayers: dict = dataclasses.field(default_factory=dict)  # name -> LayerRecord
    values: dict = dataclasses.field(default_factory=dict)  # name -> int | float
    matrices: dict = dataclasses.field(default_factory=dict)  # name -> MatrixRecord

    def sub(self, name: str) -> "LayerRecord":
        if name not in self.sublayers:
            raise CheckpointError(f"layer {self.name or self.path!r} has no sub-layer {name!r}")
        return self.sublayers[name]

    def matrix(self, name: str) -> MatrixRecord:
        if name not in self.matrices:
            raise CheckpointError(f"layer {self.name or self.path!r} has no matrix {name!r}")
        return self.matrices[name]


@dataclasses.dataclass
class Checkpoint:
    path: str
    layers: list  # LayerRecord in model.guide order
    input_dims: tuple | None
    optimiser: str | None
    loss: str | None

    def layer(self, name: str) -> LayerRecord:
        for rec in self.layers:
            if rec.name == name:
                return rec
        raise CheckpointError(f"{self.path}: no layer named {name!r}")


def _records(path: str):
    """(NAME, DATA, TYPE, META, GUID) records of a text blob file; ';' closes a record and a
    trailing record without one is kept, as SaveLoader.h:676-781 does."""
    try:
        with open(path, "r") as f:
            lines = f.read().splitlines()
    except OSError as e:
        raise CheckpointError(f"cannot read {path}: {e}") from None
    cur: dict = {}
    out = []
    for line in lines:
        line = line.strip()
        if not line:
            continue
        if line == ";":
            if cur.get("NAME"):
                out.append(cur)
            cur = {}
            continue
        key, _, val = line.partition(" ")
        if key in ("NAME", "DATA", "TYPE", "META", "GUID"):
            cur[key] = val.strip()
    if cur.get("NAME"):
        out.append(cur)
    return out


def _guid(text):
    try:
        return int(text)
    except (TypeError, ValueError):
        return None


def _read_matrix(path: str) -> MatrixRecord:
    """Key/value lines up to the first ';' (SaveLoader.h:1267-1348)."""
    try:
        with open(path, "r") as f:
            lines = f.read().splitlines()
    except OSError as e:
        raise CheckpointError(f"cannot read {path}: {e}") from None
    fields = {}
    for line in lines:
        line = line.strip()
        if line == ";":
            break
        key, _, val = line.partition(" ")
        if key:
            fields[key] = val.strip()
    if not fields.get("DATA"):
        raise CheckpointError(f"{path}: matrix file has no DATA entry")
    try:
        dims = tuple(int(fields.get(k, "0")) for k in ("DIMX", "DIMY", "DIMZ"))
    except ValueError:
        raise CheckpointError(f"{path}: bad DIMX/DIMY/DIMZ") from None
    return MatrixRecord(path, fields.get("INTERNAL_NAME", ""), _guid(fields.get("GUID")), dims,
                        os.path.join(os.path.dirname(path), fields["DATA"]))


def _read_value(path: str, kind: str):
    raw = np.fromfile(path, dtype=np.uint8)
    if raw.size != 4:
        raise CheckpointError(f"{path}: {kind} value file holds {raw.size} bytes, expected 4")
    dt = {"INT": "<i4", "UINT": "<u4", "FLOAT": "<f4"}[kind]
    v = raw.view(dt)[0]
    return float(v) if kind == "FLOAT" else int(v)


def read_layer(path: str) -> LayerRecord:
    """Parse one ``.blob_layer`` file and, recursively, its sub-layers."""
    base = os.path.dirname(path)
    rec = LayerRecord(path)
    for r in _records(path):
        name, data, typ = r.get("NAME", ""), r.get("DATA", ""), r.get("TYPE", "")
        if name == "Layer_Name":
            rec.name, rec.meta, rec.guid = data, r.get("META", ""), _guid(r.get("GUID"))
            rec.type = typ[len("ROOTLAYER_"):] if typ.startswith("ROOTLAYER_") else typ
        elif typ.startswith("LAYER_") or typ.startswith("ROOTLAYER_"):
            sub = read_layer(os.path.join(base, data))
            if not sub.type:
                sub.type = typ.split("_", 1)[1]
            rec.sublayers[name] = sub
        elif typ in ("INT", "UINT", "FLOAT"):
            rec.values[name] = _read_value(os.path.join(base, data), typ)
        elif typ == "MATRIX":
            rec.matrices[name] = _read_matrix(os.path.join(base, data))
    return rec


def read_checkpoint(path: str) -> Checkpoint:
    """Read the model folder ``path`` (the one holding ``model.guide``)."""
    guide = os.path.join(path, "model.guide")
    if not os.path.isfile(guide):
        raise CheckpointError(f"{path}: no model.guide (not a FreeML checkpoint folder)")
    layers, dims, opt, loss = [], None, None, None
    with open(guide, "r") as f:
        for line in f:
            parts = line.split()
            if not parts:
                continue
            tag = parts[0]
            if tag == "LAYER" and len(parts) >= 3:
                layers.append(read_layer(os.path.join(path, parts[2])))
            elif tag == "INPUT_DIMS" and len(parts) >= 4:
                dims = tuple(int(v) for v in parts[1:4])
            elif tag == "OPTIMISER" and len(parts) >= 2:
                opt = None if parts[1] == "0" else os.path.join(path, parts[1])
            elif tag == "LOSSFUNC" and len(parts) >= 2:
                loss = None if parts[1] == "0" else os.path.join(path, parts[1])
    if not layers:
        raise CheckpointError(f"{guide}: no LAYER lines")
    return Checkpoint(path, layers, dims, opt, loss)


def _vec(m: MatrixRecord, n: int, what: str) -> np.ndarray:
    a = m.array().reshape(-1)
    if a.size != n:
        raise CheckpointError(f"{what}: {a.size} values, expected {n}")
    return np.ascontiguousarray(a)


def _mat(m: MatrixRecord, rows: int, cols: int, what: str) -> np.ndarray:
    if m.dims != (cols, rows, 1):
        raise CheckpointError(f"{what}: dims {m.dims}, expected ({cols}, {rows}, 1)")
    return np.ascontiguousarray(m.array().reshape(rows, cols))


def load_nanollm(path: str) -> NanoLLMWeights:
    """NanoLLM parameters from a checkpoint folder, in the storage layout ``NanoLLM`` uploads.

    The graph must be NanoLLM.cpp:267-358's: ``embedding_token``, ``embedding_pos``,
    ``block_0..L-1`` (TransformerBlock), ``ln_f`` (LayerNorm) and ``lm_head`` (Dense).  The
    shape comes from the matrices (vocab and n_embed from embedding_token's {C, V} weights,
    block_size from embedding_pos's {C, T}) and n_head from the attention blob's
    ``NumHeads``.  lm_head is tied when its ``Dense_Weights`` carries the embedding's GUID.
    Dense biases (NanoLLM ``use_bias``) are refused: the device graph has none.
    """
    ck = read_checkpoint(path)
    types = {"embedding_token": "Embedding", "embedding_pos": "Embedding", "ln_f": "LayerNorm",
             "lm_head": "Dense"}
    for name, typ in types.items():
        if ck.layer(name).type != typ:
            raise CheckpointError(f"{path}: layer {name!r} is {ck.layer(name).type}, expected {typ}")
    blocks = []
    while any(r.name == f"block_{len(blocks)}" for r in ck.layers):
        b = ck.layer(f"block_{len(blocks)}")
        if b.type != "TransformerBlock":
            raise CheckpointError(f"{path}: {b.name} is {b.type}, expected TransformerBlock")
        blocks.append(b)
    if not blocks:
        raise CheckpointError(f"{path}: no TransformerBlock layers block_0..")

    tok_m = ck.layer("embedding_token").matrix("Embedding_Weights")
    pos_m = ck.layer("embedding_pos").matrix("Embedding_Weights")
    C, V = tok_m.dims[0], tok_m.dims[1]
    T = pos_m.dims[1]
    heads = {b.sub("AttentionLayerData").values.get("NumHeads") for b in blocks}
    if len(heads) != 1 or None in heads:
        raise CheckpointError(f"{path}: NumHeads missing or differing across blocks: {heads}")
    H = heads.pop()
    if H <= 0 or C % H:
        raise CheckpointError(f"{path}: n_embed {C} not divisible by NumHeads {H}")

    head = ck.layer("lm_head")
    head_m = head.matrix("Dense_Weights")
    tied = head_m.guid is not None and head_m.guid == tok_m.guid
    shape = NanoLLMShape(V, T, C, H, len(blocks), tied=tied)

    def ln(rec: LayerRecord, what: str):
        g = _vec(rec.matrix("GammaScale"), C, what + " GammaScale")
        b = rec.matrices.get("BetaShift")
        return g, (_vec(b, C, what + " BetaShift") if b is not None else None)

    layers = []
    for l, b in enumerate(blocks):
        att = b.sub("AttentionLayerData")
        qkv, proj = att.sub("CSA_AttentionLayer"), att.sub("CSA_ProjLayer")
        fc, pr = b.sub("DenseFCData"), b.sub("DenseProjData")
        for d in (qkv, proj, fc, pr):
            if "Dense_Bias" in d.matrices:
                raise CheckpointError(f"{path}: block_{l} has Dense_Bias (use_bias); unsupported")
        g0, b0 = ln(b.sub("LayerNorm0Data"), f"block_{l} LayerNorm0")
        g1, b1 = ln(b.sub("LayerNorm1Data"), f"block_{l} LayerNorm1")
        layers.append(LayerWeights(
            w_qkv=_mat(qkv.matrix("Dense_Weights"), C, 3 * C, f"block_{l} qkv"),
            w_proj=_mat(proj.matrix("Dense_Weights"), C, C, f"block_{l} proj"),
            w_fc=_mat(fc.matrix("Dense_Weights"), C, 4 * C, f"block_{l} fc"),
            w_proj2=_mat(pr.matrix("Dense_Weights"), 4 * C, C, f"block_{l} proj2"),
            ln0_g=g0, ln1_g=g1, ln0_b=b0, ln1_b=b1))
    if "Dense_Bias" in head.matrices:
        raise CheckpointError(f"{path}: lm_head has Dense_Bias (use_bias); unsupported")
    lnf_g, lnf_b = ln(ck.layer("ln_f"), "ln_f")
    tok = _mat(tok_m, V, C, "embedding_token")
    lm = tok if tied else _mat(head_m, V, C, "lm_head")
    return NanoLLMWeights(shape, tok, _mat(pos_m, T, C, "embedding_pos"), layers, lnf_g, lnf_b, lm)
