"""Variable-length packed spectral KV cache (drop-in ``CustomDynamicCache``).

Mirrors the reference ``src/dynakv/kernels/compressed_cache.py:58-227``. Per layer and per K/V
the cache holds the list ``[flat, lens, offs, ptr, seq, ub]``:

* ``flat``  ``(rows, cap_flat)`` packed coefficients in the states' dtype, zero outside
  ``[0, ptr[b])``;
* ``lens``/``offs`` ``(rows, cap_seq)`` int32; ``offs`` is the exclusive prefix sum of ``lens``;
* ``ptr``   ``(rows,)`` int32 on the device, next free element of each row;
* ``seq``   host int, number of tokens stored;
* ``ub``    host list, an upper bound of ``ptr`` that lets decode steps skip device reads.

The capacity policy is the reference's, so buffer shapes match it exactly:
sequence capacity grows to ``max(cap + 1024, seq + new)``; on a decode step the flat capacity
is checked against ``max(ub) + new * max_dim`` and only then is ``ptr`` read back; growth goes to
``max(cap + 1024 * (max_dim // 2), max(ptr) + added)``. Device work (append, prefill packing,
re-expansion) runs in the gfx950 kernels of ``libdynakv_amd``; the decode step issues one
launch for K and V together.
"""

from __future__ import annotations

from typing import Optional

import torch

from .. import _lib

try:  # the HF cache base class keeps the object usable where transformers expects a Cache
    from transformers.cache_utils import DynamicCache as _CacheBase
except Exception:  # pragma: no cover - transformers is optional for the kernels
    _CacheBase = object

EXPAND_SEQ_STEP = 1024


def _max_dim_of(tensor_d) -> int:
    if isinstance(tensor_d, torch.Tensor):
        return int(tensor_d.max().item())
    return int(tensor_d)


def seq_capacity_after(cap_seq: int, seq: int, new_s: int) -> int:
    """Sequence-table capacity after adding ``new_s`` tokens (reference :135-145)."""
    if seq + new_s > cap_seq:
        return max(cap_seq + EXPAND_SEQ_STEP, seq + new_s)
    return cap_seq


def flat_capacity_after(cap_flat: int, real_ptrs: list[int], added: int, max_dim: int) -> int:
    """Flat capacity once the true pointers are known (reference :158-168)."""
    if max(real_ptrs) + added > cap_flat:
        return max(cap_flat + EXPAND_SEQ_STEP * (max_dim // 2), max(real_ptrs) + added)
    return cap_flat


class CustomDynamicCache(_CacheBase):
    def __init__(self, config=None, max_batch_size=None, max_cache_len=None, dtype=None,
                 device=None, layer_device_map=None, **kwargs):
        if _CacheBase is not object:
            super().__init__()
        # kept under the reference's names (it stores them and never reads them)
        self.max_batch_size = max_batch_size
        self.max_cache_len = max_cache_len
        self.dtype = dtype
        self.device = device
        self.layer_device_map = layer_device_map
        self.key_cache_sp: list = []
        self.value_cache_sp: list = []
        self.device_syncs = 0  # host reads of device state (growth checks, prefill bounds)

    # transformers 5 makes these read-only (deprecated) properties of its Cache class; the
    # reference's cache assigns them in its constructor (compressed_cache.py:61-62), so they are
    # plain stored values here
    @property
    def max_batch_size(self):
        return self._max_batch_size

    @max_batch_size.setter
    def max_batch_size(self, value):
        self._max_batch_size = value

    @property
    def max_cache_len(self):
        return self._max_cache_len

    @max_cache_len.setter
    def max_cache_len(self, value):
        self._max_cache_len = value

    # ------------------------------------------------------------------ queries
    def get_origin_states(self, max_dim, layer_idx):
        """Dense ``(rows, seq, max_dim)`` K and V coefficients (reference :70-81)."""
        c_k = self.key_cache_sp[layer_idx]
        c_v = self.value_cache_sp[layer_idx]
        return self._decompress(c_k, max_dim), self._decompress(c_v, max_dim)

    def reset(self):
        self.key_cache_sp = []
        self.value_cache_sp = []

    def get_seq_length_sp(self, layer_idx: Optional[int] = 0) -> int:
        if len(self.key_cache_sp) <= layer_idx:
            return 0
        if self.key_cache_sp[layer_idx] is None:
            return 0
        return self.key_cache_sp[layer_idx][4]

    def get_seq_length(self, layer_idx: Optional[int] = 0) -> int:
        """Expose the compressed sequence length through the HF Cache API."""
        return self.get_seq_length_sp(layer_idx)

    # ------------------------------------------------------------------ updates
    def _prepare_slot(self, cache_list, layer_idx, new_states, new_len, max_dim, is_decode,
                      row_max=None):
        """Host-side bookkeeping of one slot; returns ``(cache, added)`` ready for the kernel.
        ``row_max``: max over rows of the summed new lengths when the caller already has it
        (a prefill append then needs no device synchronisation of its own)."""
        while len(cache_list) <= layer_idx:
            cache_list.append(None)
        B, new_s = new_len.shape
        added = None if row_max is None else int(row_max)
        if cache_list[layer_idx] is None:
            if added is None:
                init_flat = int(new_len.sum(dim=1).max().item())
                self.device_syncs += 1
            else:
                init_flat = added
            if not is_decode:
                added = init_flat  # the same reduction sizes the append below
            flat = new_states.new_zeros(B, init_flat)
            lens = torch.zeros(B, new_s, dtype=torch.int32, device=new_len.device)
            offs = torch.zeros(B, new_s, dtype=torch.int32, device=new_len.device)
            ptr = torch.zeros(B, dtype=torch.int32, device=new_states.device)
            cache_list[layer_idx] = [flat, lens, offs, ptr, 0, [0] * B]
        cache = cache_list[layer_idx]
        flat, lens, offs, ptr, seq, ub = cache

        new_cap = seq_capacity_after(lens.shape[1], seq, new_s)
        if new_cap != lens.shape[1]:
            nl = lens.new_zeros(B, new_cap)
            nl[:, :seq].copy_(lens[:, :seq])
            no = offs.new_zeros(B, new_cap)
            no[:, :seq].copy_(offs[:, :seq])
            cache[1], cache[2] = nl, no

        if is_decode:
            added = new_s * max_dim
        elif added is None:
            added = int(new_len.sum(dim=1).max().item())
            self.device_syncs += 1
        if max(ub) + added > flat.shape[1]:
            real = ptr.cpu().tolist()
            self.device_syncs += 1
            cache[5] = real
            cap = flat_capacity_after(flat.shape[1], real, added, max_dim)
            if cap != flat.shape[1]:
                nf = flat.new_zeros(B, cap)
                # beyond ptr[b] the old buffer is zero, so one block copy equals the per-row
                # prefix copies of the reference
                nf[:, : flat.shape[1]].copy_(flat)
                cache[0] = nf
        return cache, added

    def _finish_slot(self, cache, new_s, added, is_decode):
        cache[4] = cache[4] + new_s
        if is_decode:
            cache[5] = [p + added for p in cache[5]]

    def _launch_prefill_pair(self, ck, ks, kl, ub_k, cv, vs, vl, ub_v, max_dim):
        """The prefill appends of a layer's K and V slots: one ``dkv_append_prefill_kv`` launch
        when both slots stand at the same length with the same rows, tokens and dtype, else one
        ``dkv_append_prefill`` per slot (the same results)."""
        if (ck[4] != cv[4] or ck[0].dtype != cv[0].dtype or tuple(kl.shape) != tuple(vl.shape)
                or tuple(ks.shape) != tuple(vs.shape)):
            self._launch_prefill(ck, ks, kl, max_dim, ub=ub_k)
            self._launch_prefill(cv, vs, vl, max_dim, ub=ub_v)
            return
        fk, lk, okk, pk, seq, _ = ck
        fv, lv, ov, pv, _, _ = cv
        sk = ks if ks.stride(-1) == 1 else ks.contiguous()
        sv = vs if vs.stride(-1) == 1 else vs.contiguous()
        nk, nv = kl.to(torch.int32), vl.to(torch.int32)
        B, new_s = kl.shape
        rc = _lib.load().dkv_append_prefill_kv(
            _lib.stream_of(fk), _lib.dtype_code(fk.dtype), seq, B, new_s, max_dim,
            sk.data_ptr(), sk.stride(0), sk.stride(1), nk.data_ptr(), nk.stride(0), nk.stride(1),
            fk.data_ptr(), fk.stride(0), lk.data_ptr(), okk.data_ptr(), lk.stride(0),
            lk.stride(1), pk.data_ptr(),
            sv.data_ptr(), sv.stride(0), sv.stride(1), nv.data_ptr(), nv.stride(0), nv.stride(1),
            fv.data_ptr(), fv.stride(0), lv.data_ptr(), ov.data_ptr(), lv.stride(0),
            lv.stride(1), pv.data_ptr())
        _lib.check(rc, "dkv_append_prefill_kv")
        for cache, ub in ((ck, ub_k), (cv, ub_v)):
            if ub is not None:
                cache[5] = [int(v) for v in ub]
            else:
                cache[5] = cache[3].cpu().tolist()
                self.device_syncs += 1

    def _launch_prefill(self, cache, new_states, new_len, max_dim, ub=None):
        """``ub``: the rows' pointers after the append when the caller knows them (a slot
        that started empty); otherwise they are read back from the device."""
        flat, lens, offs, ptr, seq, _ = cache
        B, new_s = new_len.shape
        st = _lib.stream_of(flat)
        states = new_states if new_states.stride(-1) == 1 else new_states.contiguous()
        nl = new_len.to(torch.int32)
        rc = _lib.load().dkv_append_prefill(
            st, _lib.dtype_code(flat.dtype), states.data_ptr(), states.stride(0), states.stride(1),
            nl.data_ptr(), nl.stride(0), nl.stride(1), flat.data_ptr(), flat.stride(0),
            lens.data_ptr(), offs.data_ptr(), lens.stride(0), lens.stride(1),
            ptr.data_ptr(), seq, B, new_s, max_dim)
        _lib.check(rc, "dkv_append_prefill")
        if ub is not None:
            cache[5] = [int(v) for v in ub]
        else:
            cache[5] = ptr.cpu().tolist()
            self.device_syncs += 1

    @staticmethod
    def _decode_view(new_states, new_len):
        states = new_states.reshape(new_states.shape[0], -1)
        if states.stride(1) != 1:
            states = states.contiguous()
        nl = new_len.to(torch.int32)
        return states, nl

    def _update_layer_cache(self, cache_list, layer_idx, new_states, new_len, tensor_d,
                            is_decode=False):
        max_dim = _max_dim_of(tensor_d)
        cache, added = self._prepare_slot(cache_list, layer_idx, new_states, new_len, max_dim,
                                          is_decode)
        if is_decode:
            flat, lens, offs, ptr, seq, _ = cache
            states, nl = self._decode_view(new_states, new_len)
            rc = _lib.load().dkv_append_decode(
                _lib.stream_of(flat), _lib.dtype_code(flat.dtype), states.data_ptr(),
                states.stride(0), nl.data_ptr(), nl.stride(0), flat.data_ptr(), flat.stride(0),
                lens.data_ptr(), offs.data_ptr(), lens.stride(0), lens.stride(1), ptr.data_ptr(),
                seq, new_len.shape[0], max_dim)
            _lib.check(rc, "dkv_append_decode")
        else:
            self._launch_prefill(cache, new_states, new_len, max_dim)
        self._finish_slot(cache, new_len.shape[1], added, is_decode)

    def update_sp_prefill_many(self, items, tensor_d):
        """Prefill appends of several layers, ``items`` = [(layer_idx, key_states, key_len,
        value_states, value_len), ...] (each as ``update_sp`` takes them, S > 1): the same
        cache state as one ``update_sp`` per layer, with one device synchronisation for all
        of them (the per-row length totals that size each slot's buffer) instead of one per
        slot."""
        if not items:
            return
        max_dim = _max_dim_of(tensor_d)
        lens = [l for it in items for l in (it[2], it[4])]
        if any(it[1].shape[1] == 1 for it in items):
            raise ValueError("update_sp_prefill_many takes prefill appends (S > 1)")
        # per slot and row: the summed counts (buffer sizing) and the clipped sums (the row's
        # pointer after the append, for a slot that starts empty), in one transfer
        if len({tuple(l.shape) for l in lens}) == 1:
            L = torch.stack(lens)  # one reduction over every slot instead of one per slot
            host = torch.cat([L.sum(dim=2).flatten(),
                              L.clamp(0, max_dim).sum(dim=2).flatten()]).tolist()
        else:
            host = torch.cat([l.sum(dim=1) for l in lens] +
                             [l.clamp(0, max_dim).sum(dim=1) for l in lens]).tolist()
        self.device_syncs += 1
        rows = [l.shape[0] for l in lens]
        starts = [sum(rows[:k]) for k in range(len(lens))]
        half = sum(rows)
        created = self._create_fresh_slots(items, lens, host, starts)
        for n, (layer_idx, ks, kl, vs, vl) in enumerate(items):
            prepared = []
            for j, (cache_list, st, ln) in enumerate(((self.key_cache_sp, ks, kl),
                                                      (self.value_cache_sp, vs, vl))):
                k = 2 * n + j
                su = host[starts[k]:starts[k] + rows[k]]
                sc = host[half + starts[k]:half + starts[k] + rows[k]]
                fresh = (j, layer_idx) in created or (len(cache_list) <= layer_idx
                                                      or cache_list[layer_idx] is None)
                cache, added = self._prepare_slot(cache_list, layer_idx, st, ln, max_dim, False,
                                                  row_max=max(su))
                prepared.append((cache, st, ln, added, sc if fresh else None))
            (ck, kst, kln, kadd, kub), (cv, vst, vln, vadd, vub) = prepared
            self._launch_prefill_pair(ck, kst, kln, kub, cv, vst, vln, vub, max_dim)
            self._finish_slot(ck, kln.shape[1], kadd, False)
            self._finish_slot(cv, vln.shape[1], vadd, False)

    def _create_fresh_slots(self, items, lens, host, starts):
        """The slots of ``items`` that do not exist yet, created as ``_prepare_slot`` creates
        them (flat sized to the largest row total, tables to the prompt, pointers zero) but
        from one zeroed buffer for every flat and pointer array and one unfilled buffer for the
        tables (the prefill append writes every table entry of a fresh slot): two fills in all
        instead of four per slot. Returns the created slots as ``(0 (K) | 1 (V), layer)``;
        a slot whose rows hold no coefficient at all is left to ``_prepare_slot``."""
        fresh = []
        for n, it in enumerate(items):
            layer_idx = it[0]
            for j, (cache_list, st) in enumerate(((self.key_cache_sp, it[1]),
                                                  (self.value_cache_sp, it[3]))):
                while len(cache_list) <= layer_idx:
                    cache_list.append(None)
                if cache_list[layer_idx] is None:
                    k = 2 * n + j
                    cap = max(host[starts[k]:starts[k] + lens[k].shape[0]])
                    if cap > 0:
                        fresh.append((cache_list, layer_idx, st, lens[k], cap, j))
        if not fresh:
            return set()
        dev = fresh[0][2].device
        by_dtype = {}
        for f in fresh:
            by_dtype.setdefault(f[2].dtype, []).append(f)
        tab_elems = sum(f[3].numel() for f in fresh)
        tabs = torch.empty(2 * tab_elems, dtype=torch.int32, device=dev)
        ptrs = torch.zeros(sum(f[3].shape[0] for f in fresh), dtype=torch.int32, device=dev)
        t_at = p_at = 0
        for dt, group in by_dtype.items():
            flats = torch.zeros(sum(f[3].shape[0] * f[4] for f in group), dtype=dt, device=dev)
            f_at = 0
            for cache_list, layer_idx, st, ln, cap, _ in group:
                B, S = ln.shape
                flat = flats[f_at:f_at + B * cap].view(B, cap)
                f_at += B * cap
                lt = tabs[t_at:t_at + B * S].view(B, S)
                ot = tabs[tab_elems + t_at:tab_elems + t_at + B * S].view(B, S)
                t_at += B * S
                ptr = ptrs[p_at:p_at + B]
                p_at += B
                cache_list[layer_idx] = [flat, lt, ot, ptr, 0, [0] * B]
        return {(f[5], f[1]) for f in fresh}

    def update_sp(self, key_states, key_len, value_states, value_len, max_dim, layer_idx,
                  tensor_d, k_scalar=None, v_scalar=None):
        """Append K and V coefficients of ``layer_idx`` (reference :219-227).

        Decode (``key_states.shape[1] == 1``) issues a single launch for both slots.
        Returns ``(flat_k, flat_v, lens_k, lens_v, offs_k, offs_v)`` with the tables cut to the
        stored length.
        """
        is_decode = key_states.shape[1] == 1
        if is_decode:
            md = _max_dim_of(tensor_d)
            ck, add_k = self._prepare_slot(self.key_cache_sp, layer_idx, key_states, key_len, md, True)
            cv, add_v = self._prepare_slot(self.value_cache_sp, layer_idx, value_states, value_len,
                                           md, True)
            if ck[4] != cv[4] or ck[0].dtype != cv[0].dtype:
                # K and V slots out of step: fall back to one launch each
                self._launch_decode_single(ck, key_states, key_len, md)
                self._launch_decode_single(cv, value_states, value_len, md)
            else:
                ks, kl = self._decode_view(key_states, key_len)
                vs, vl = self._decode_view(value_states, value_len)
                fk, lk, ok, pk, seq, _ = ck
                fv, lv, ov, pv, _, _ = cv
                rc = _lib.load().dkv_append_decode_kv(
                    _lib.stream_of(fk), _lib.dtype_code(fk.dtype), key_len.shape[0], md, seq,
                    ks.data_ptr(), ks.stride(0), kl.data_ptr(), kl.stride(0),
                    fk.data_ptr(), fk.stride(0), lk.data_ptr(), ok.data_ptr(),
                    lk.stride(0), lk.stride(1), pk.data_ptr(),
                    vs.data_ptr(), vs.stride(0), vl.data_ptr(), vl.stride(0),
                    fv.data_ptr(), fv.stride(0), lv.data_ptr(), ov.data_ptr(),
                    lv.stride(0), lv.stride(1), pv.data_ptr())
                _lib.check(rc, "dkv_append_decode_kv")
            self._finish_slot(ck, key_len.shape[1], add_k, True)
            self._finish_slot(cv, value_len.shape[1], add_v, True)
        else:
            self._update_layer_cache(self.key_cache_sp, layer_idx, key_states, key_len, tensor_d,
                                     is_decode=False)
            self._update_layer_cache(self.value_cache_sp, layer_idx, value_states, value_len,
                                     tensor_d, is_decode=False)
        c_k = self.key_cache_sp[layer_idx]
        c_v = self.value_cache_sp[layer_idx]
        return (c_k[0], c_v[0], c_k[1][:, : c_k[4]], c_v[1][:, : c_v[4]],
                c_k[2][:, : c_k[4]], c_v[2][:, : c_v[4]])

    def _launch_decode_single(self, cache, new_states, new_len, max_dim):
        flat, lens, offs, ptr, seq, _ = cache
        states, nl = self._decode_view(new_states, new_len)
        rc = _lib.load().dkv_append_decode(
            _lib.stream_of(flat), _lib.dtype_code(flat.dtype), states.data_ptr(), states.stride(0),
            nl.data_ptr(), nl.stride(0), flat.data_ptr(), flat.stride(0), lens.data_ptr(),
            offs.data_ptr(), lens.stride(0), lens.stride(1), ptr.data_ptr(), seq,
            new_len.shape[0], max_dim)
        _lib.check(rc, "dkv_append_decode")

    def _decompress(self, cache, max_dim):
        flat, lens, offs, _, seq, _ = cache
        rows = flat.shape[0]
        out = flat.new_empty(rows, seq, max_dim)
        if rows == 0 or seq == 0:
            return out.zero_()
        rc = _lib.load().dkv_decompress(
            _lib.stream_of(flat), _lib.dtype_code(flat.dtype), flat.data_ptr(), flat.stride(0),
            lens.data_ptr(), offs.data_ptr(), lens.stride(0), lens.stride(1), out.data_ptr(),
            rows, seq, max_dim)
        _lib.check(rc, "dkv_decompress")
        return out
