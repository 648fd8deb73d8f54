'use strict';
// MI355X drop-in for the LFM2-MoE MoE feed-forward path of QwenQwen3.js.
//
// Keeps the reference's JavaScript call surface and runs it on the gfx950 HIP
// library through the Node-API addon (qq_napi.node -> libqqmoe.so):
//   matmulQ80xF32(meta, input)      src/tensor.js:26-53
//   matmulGeneric(meta, input)      src/tensor.js:485-496 (type 8; other types are
//                                   delegated to the matmulGeneric being replaced)
//   Lfm2Engine.prototype._moEFFN    src/lfm2-engine.js:413-487 (sigmoid + bias gating)
//   Qwen3Engine.prototype._moEFFN   src/qwen3-engine.js:304-363 (softmax gating)
// plus entry points with no reference counterpart:
//   device.moeForward(layer, X, hidden, T, {mask, wantProbs})   T tokens at once
//   device.attachGGUF(path)   MoE blocks come from the file (memory-mapped,
//                             repacked straight to the device) instead of from
//                             the engine's ArrayBuffers
//   device.attachLfm2Forward(engine)   Lfm2Engine.forward / resetState
//                             (src/lfm2-engine.js:216-280) of one engine run the
//                             whole token on the device from the attached file,
//                             honouring engine.expertMask and calling
//                             engine.onRouterUpdate for every MoE block
// and, for hosts that keep activations in device memory as the WebGPU engines
// do (src/webgpu.js):
//   device.createBuffer / uploadBuffer / writeBuffer / readF32   GPUDevice's buffer
//                             calls (src/webgpu.js:369-430) on DeviceBuffers
//   Lfm2GPUEngine.prototype._moEFFNGPU, Qwen3GPUEngine.prototype._moEFFNGPU and
//   their _readbackRoutingData (src/webgpu.js:1882-1945, :878-990), for engines
//                             whose buffers are this device's
//   device.moeForwardDev / matvecDev / rmsnormDev   the *_dev entry points
//
// There is no CPU fallback: when the addon or the device is missing, the
// constructor and install() throw.  Written for Node 12 (no `?.`, no `??`).

const path = require('path');

const ADDON_PATH = path.join(__dirname, '..', 'qq_napi.node');
let addon = null;

function native() {
    if (!addon) addon = require(ADDON_PATH);
    return addon;
}

function halfToNumber(bits) {
    const sign = (bits & 0x8000) ? -1 : 1;
    const exp = (bits >>> 10) & 0x1f;
    const man = bits & 0x3ff;
    if (exp === 0) return sign * man * Math.pow(2, -24);
    if (exp === 31) return man ? NaN : sign * Infinity;
    return sign * (1024 + man) * Math.pow(2, exp - 25);
}

// _readWeightF32 (src/tensor.js:80-100) for the expert-bias vector.
function readWeightF32(meta, n) {
    if (meta.type === 0) return new Float32Array(meta.buffer, meta.offset, n).slice();
    if (meta.type === 8) {
        const u8 = new Uint8Array(meta.buffer), i8 = new Int8Array(meta.buffer);
        const out = new Float32Array(n);
        for (let b = 0; b < Math.ceil(n / 32); b++) {
            const p = meta.offset + b * 34;
            const d = halfToNumber(u8[p] | (u8[p + 1] << 8));
            for (let i = 0; i < 32 && b * 32 + i < n; i++) out[b * 32 + i] = i8[p + 2 + i] * d;
        }
        return out;
    }
    throw new Error('Unsupported weight type for norm: ' + meta.type);
}

const GATING_SIGMOID_BIAS = 0;   // LFM2-MoE
const GATING_SOFTMAX = 1;        // Qwen3-MoE

function asFloat32(a) {
    return (a instanceof Float32Array) ? a : Float32Array.from(a);
}

// Device memory standing for a WebGPU GPUBuffer (src/webgpu.js:369-392), or a
// byte range of one: views share their root's allocation, which release()
// (or garbage collection) frees.
class DeviceBuffer {
    constructor(device, handle, byteOffset, size, root) {
        this.device = device;
        this.handle = handle;
        this.byteOffset = byteOffset;
        this.size = size;
        this.root = root || null;
    }

    view(byteOffset, size) {
        if (byteOffset < 0 || size < 0 || byteOffset + size > this.size || (byteOffset & 3))
            throw new RangeError('DeviceBuffer.view: [' + byteOffset + ', +' + size + ') outside ' + this.size + ' bytes');
        return new DeviceBuffer(this.device, this.handle, this.byteOffset + byteOffset, size, this.root || this);
    }

    release() {
        if (!this.root && this.handle) this.device.native.release(this.handle);
        this.handle = null;
    }
}

function engineDims(eng) {
    // Lfm2GPUEngine keeps the CPU engine's configuration in _cpu
    // (src/webgpu.js:1470-1500); Qwen3GPUEngine holds it itself (:498-530)
    const c = eng._cpu && eng._cpu.nExperts ? eng._cpu : eng;
    return { E: c.nExperts, K: c.nExpertsUsed };
}

class MoEDevice {
    constructor(device) {
        this.native = native();
        this.ctx = this.native.init(device === undefined ? 0 : (device | 0));
        this._tensors = new WeakMap();   // ArrayBuffer -> Map(key -> device tensor)
        this.fallbackMatmul = null;
        this._gguf = null;
        this._lfm2 = [];                 // {engine, model}: one device model per engine
        // GPUDevice.device.queue.writeBuffer (src/webgpu.js:1966), for engines
        // whose _gpu is this device
        const dev = this;
        this.device = { queue: { writeBuffer: function (buf, off, data) { dev.writeBuffer(buf, off, data); } } };
        // device-side waits reported as timed out by this device's synchronising
        // calls: an engine whose residual stream lives here is invalid after one
        this.timeouts = 0;
    }

    // A synchronising native call; counts a reported device-side timeout.
    _sync(f) {
        try {
            return f();
        } catch (e) {
            if (/timed out/.test(String(e && e.message))) this.timeouts++;
            throw e;
        }
    }

    // ---- device buffers: GPUDevice.createBuffer / uploadBuffer / readF32 ----
    // (src/webgpu.js:369-430): sizes round up to 4 bytes, memory starts zeroed.
    createBuffer(size) {
        const n = Math.ceil(size / 4) * 4;
        return new DeviceBuffer(this, this.native.bufAlloc(this.ctx, n), 0, n, null);
    }

    uploadBuffer(data) {
        const bytes = data instanceof ArrayBuffer ? new Uint8Array(data)
                    : new Uint8Array(data.buffer, data.byteOffset, data.byteLength);
        const buf = this.createBuffer(bytes.length);
        this.writeBuffer(buf, 0, bytes);
        return buf;
    }

    writeBuffer(buf, byteOffset, data) {
        this._own(buf, 'writeBuffer');
        const dev = this;
        this._sync(function () { dev.native.bufWrite(dev.ctx, buf.handle, buf.byteOffset + (byteOffset | 0), data); });
    }

    // The values once the work enqueued before the call has run.
    readF32Sync(buf, nElems, byteOffset) {
        this._own(buf, 'readF32');
        const out = new Float32Array(nElems);
        const dev = this;
        this._sync(function () { dev.native.bufRead(dev.ctx, buf.handle, buf.byteOffset + (byteOffset | 0), out); });
        return out;
    }

    readF32(buf, nElems) {
        const dev = this;
        return new Promise(function (resolve) { resolve(dev.readF32Sync(buf, nElems)); });
    }

    // Bound on the batch-1 decode kernel's device-side waits (qq_set_wait_limit).
    setWaitLimit(microseconds) { this.native.setWaitLimit(this.ctx, microseconds | 0); }

    synchronize() {
        const dev = this;
        this._sync(function () { dev.native.synchronize(dev.ctx); });
    }

    _own(buf, what) {
        if (!(buf instanceof DeviceBuffer) || buf.device !== this || !buf.handle)
            throw new TypeError(what + ': expected a live DeviceBuffer of this device');
    }

    // ---- device-pointer calls (include/qq_moe.h *_dev), enqueued ----
    // hidden += MoE(x) for T rows of device buffers; opts as moeForward plus
    // record: a DeviceBuffer receiving the routing record of every row
    // ([K experts | K weights | E probs] as floats, qq_moe_forward_record_dev).
    moeForwardDev(layer, xBuf, hiddenBuf, T, opts) {
        const o = opts || {};
        const K = o.K !== undefined ? o.K : 4;
        const E = layer.ffnGateExps.shape[2];
        const h = this.layerHandle(layer, E, K, o.gating, o.block);
        let mask = null;
        if (o.mask && o.mask.size) {
            mask = new Uint8Array(h.E);
            o.mask.forEach(function (e) { if (e >= 0 && e < h.E) mask[e] = 1; });
        }
        this._own(xBuf, 'moeForwardDev');
        this._own(hiddenBuf, 'moeForwardDev');
        const rec = o.record || null;
        if (rec) this._own(rec, 'moeForwardDev');
        this.native.moeForwardDev(this.ctx, h.moe, xBuf.handle, xBuf.byteOffset, hiddenBuf.handle,
                                  hiddenBuf.byteOffset, T | 0, mask, rec ? rec.handle : null, rec ? rec.byteOffset : 0);
    }

    // y = W x for `rows` vectors of device buffers (matmulQ80xF32 on device memory)
    matvecDev(meta, xBuf, yBuf, rows) {
        if (meta.type !== 8) throw new Error('matvecDev: tensor type ' + meta.type + ' is not Q8_0');
        const t = this.tensorFor(meta, meta.shape[0], meta.shape[1], 1);
        this._own(xBuf, 'matvecDev');
        this._own(yBuf, 'matvecDev');
        this.native.matvecDev(this.ctx, t, 0, xBuf.handle, xBuf.byteOffset, yBuf.handle, yBuf.byteOffset,
                              rows === undefined ? 1 : rows | 0);
    }

    // rmsnorm (src/tensor.js:103-114) of T rows of H floats; wBuf null = unit weight
    rmsnormDev(xBuf, wBuf, outBuf, T, H, eps) {
        this._own(xBuf, 'rmsnormDev');
        this._own(outBuf, 'rmsnormDev');
        if (wBuf) this._own(wBuf, 'rmsnormDev');
        this.native.rmsnormDev(this.ctx, xBuf.handle, xBuf.byteOffset, wBuf ? wBuf.handle : null,
                               wBuf ? wBuf.byteOffset : 0, outBuf.handle, outBuf.byteOffset, T | 0, H | 0, +eps);
    }

    // ---- the WebGPU engines' MoE block ----
    // True when `eng` keeps its activations in this device's buffers (its
    // _buf.normed is a DeviceBuffer of this device).
    ownsEngine(eng) {
        return !!(eng && eng._buf && eng._buf.normed instanceof DeviceBuffer && eng._buf.normed.device === this);
    }

    // Lfm2GPUEngine._moEFFNGPU / Qwen3GPUEngine._moEFFNGPU (src/webgpu.js:
    // 1882-1917, :878-915) on `eng`: _buf.hidden += MoE(_buf.normed), and the
    // routing record of MoE layer gl._moeIdx into eng._gpuRoutingBufs[moeIdx]
    // (a DeviceBuffer of 2K + E floats, made here when missing).  Enqueued: no
    // host round trip, as in the reference.  expertMask is honoured when set
    // (the WebGPU engines keep it null).
    moEFFNGPU(eng, layerIdx, gl, cl, gating) {
        // A timed-out call leaves each row of _buf.hidden old or new, and the
        // engine's other state past that point: refuse until the engine's
        // state is reset (_resetGPUState / resetKVCache, src/webgpu.js:2119)
        if (eng._qqTimeouts === undefined) eng._qqTimeouts = this.timeouts;
        if (eng._qqTimeouts !== this.timeouts)
            throw new Error('_moEFFNGPU: a device-side wait timed out since the engine\'s state was last ' +
                            'reset, so its residual stream is not valid: call resetKVCache() first');
        const d = engineDims(eng);
        const moeIdx = gl && gl._moeIdx !== undefined ? gl._moeIdx : layerIdx;
        if (!eng._gpuRoutingBufs) eng._gpuRoutingBufs = [];
        let rec = eng._gpuRoutingBufs[moeIdx];
        const recBytes = (2 * d.K + d.E) * 4;
        if (!(rec instanceof DeviceBuffer) || rec.device !== this || rec.size < recBytes) {
            rec = this.createBuffer(recBytes);
            eng._gpuRoutingBufs[moeIdx] = rec;
        }
        this.moeForwardDev(cl, eng._buf.normed, eng._buf.hidden, 1,
                           { K: d.K, gating: gating, mask: eng.expertMask, block: layerIdx, record: rec });
    }

    // _readbackRoutingData (src/webgpu.js:1922-1945, :969-990): every MoE
    // layer's routing record read back once the token's work has run (records
    // that are views of one allocation in a single read), then onRouterUpdate
    // per layer with {layer, probs, selected, weights}.
    readbackRoutingData(eng) {
        if (!eng.onRouterUpdate) return Promise.resolve();
        const d = engineDims(eng), K = d.K, E = d.E, L = 2 * K + E;
        const bufs = eng._gpuRoutingBufs || [];
        const roots = new Map();   // root allocation -> its floats, read once
        for (const b of bufs) {
            this._own(b, 'readbackRoutingData');
            const r = b.root || b;
            if (!roots.has(r)) roots.set(r, this.readF32Sync(r, r.size / 4));
        }
        for (let m = 0; m < bufs.length; m++) {
            const b = bufs[m], r = b.root || b;
            const off = (b.byteOffset - r.byteOffset) / 4;
            const res = roots.get(r).subarray(off, off + L);
            const selected = [], weights = [];
            for (let k = 0; k < K; k++) {
                selected.push(Math.round(res[k]));
                weights.push(res[K + k]);
            }
            eng.onRouterUpdate({
                layer: eng._moeAbsLayerIndices ? eng._moeAbsLayerIndices[m] : m,
                probs: Array.from(res.subarray(2 * K, 2 * K + E)),
                selected: selected,
                weights: weights,
            });
        }
        return Promise.resolve();
    }

    // Routing records of `nMoE` MoE layers as views of one allocation, so the
    // batched readback is a single copy; sets eng._gpuRoutingBufs.
    routingBuffers(eng, nMoE) {
        const d = engineDims(eng), recBytes = (2 * d.K + d.E) * 4;
        const root = this.createBuffer(recBytes * nMoE);
        const views = [];
        for (let m = 0; m < nMoE; m++) views.push(root.view(m * recBytes, recBytes));
        eng._gpuRoutingBufs = views;
        return views;
    }

    // Bind MoE blocks from a GGUF file: the layer of block l is read from the
    // file's blk.l.* tensors by the native reader (include/qq_gguf.h), which
    // maps the file instead of holding it in one ArrayBuffer (the reference
    // slices the File per tensor for the same reason, src/gguf.js:350-374).
    // Returns the file's tensor table [{name, shape, type, offset, nbytes}].
    attachGGUF(path) {
        const g = this.native.ggufOpen(String(path));
        if (this._gguf) this.native.release(this._gguf);
        this._gguf = g;
        return this.native.ggufTensors(g);
    }

    // Whole-token forward on the device (include/qq_lfm2.h) for an engine
    // whose model is the attached GGUF file: forward(tokenId, position,
    // skipLogits), resetState and resetKVCache (src/lfm2-engine.js:216-280)
    // are rebound on that engine object.  The logits land in
    // engine.bufLogits and forward returns it, or null for skipLogits, as the
    // reference does.  Returns the model's configuration (lfm2Info).
    attachLfm2Forward(engine) {
        if (!this._gguf) throw new Error('attachLfm2Forward: attachGGUF(path) first');
        const model = this.native.lfm2Create(this.ctx, this._gguf);
        // one model per engine: attaching an engine again releases only its own model
        for (let i = 0; i < this._lfm2.length; i++) {
            if (this._lfm2[i].engine === engine) {
                this.native.release(this._lfm2[i].model);
                this._lfm2.splice(i, 1);
                break;
            }
        }
        this._lfm2.push({ engine: engine, model: model });
        const info = this.native.lfm2Info(model);
        const dev = this;
        const nl = info.nLayers, K = info.nExpertsUsed, E = info.nExperts;
        const routes = { idx: new Int32Array(nl * K), w: new Float64Array(nl * K), probs: new Float32Array(nl * E) };
        const mask = new Uint8Array(E);
        if (!(engine.bufLogits instanceof Float32Array) || engine.bufLogits.length !== info.nVocab)
            engine.bufLogits = new Float32Array(info.nVocab);
        engine.forward = function (tokenId, position, skipLogits) {
            // expertMask (src/lfm2-engine.js:464): experts skipped in every MoE block
            let m = null;
            if (this.expertMask && this.expertMask.size) {
                mask.fill(0);
                this.expertMask.forEach(function (e) { if (e >= 0 && e < E) mask[e] = 1; });
                m = mask;
            }
            const want = !!this.onRouterUpdate;
            dev.native.lfm2Forward(dev.ctx, model, tokenId | 0, position | 0, skipLogits ? null : this.bufLogits,
                                   m, want ? routes : null);
            if (want) {
                // onRouterUpdate of every MoE block (src/lfm2-engine.js:449-456), with the
                // reference's payload; delivered once the token has run
                for (let l = info.nDenseLead; l < nl; l++) {
                    this.onRouterUpdate({
                        layer: l,
                        probs: Array.from(routes.probs.subarray(l * E, (l + 1) * E)),
                        selected: Array.from(routes.idx.subarray(l * K, (l + 1) * K)),
                        weights: Array.from(routes.w.subarray(l * K, (l + 1) * K)),
                    });
                }
            }
            return skipLogits ? null : this.bufLogits;
        };
        engine.resetState = function () { dev.native.lfm2Reset(dev.ctx, model); };
        engine.resetKVCache = function () { this.resetState(); };
        return info;
    }

    // Device copy of a GGUF Q8_0 tensor, uploaded (and repacked) once per
    // (buffer, offset, shape).  _expertSlice makes a new meta per call
    // (src/lfm2-engine.js:498-504), so the cache keys on the bytes, not the meta.
    tensorFor(meta, inDim, outDim, nMats) {
        let byKey = this._tensors.get(meta.buffer);
        if (!byKey) {
            byKey = new Map();
            this._tensors.set(meta.buffer, byKey);
        }
        const key = meta.offset + ':' + inDim + ':' + outDim + ':' + nMats;
        let t = byKey.get(key);
        if (!t) {
            t = this.native.uploadQ80(this.ctx, meta.buffer, meta.offset, inDim, outDim, nMats);
            byKey.set(key, t);
        }
        return t;
    }

    matmulQ80xF32(meta, input) {
        if (meta.type !== 8) throw new Error('matmulQ80xF32: tensor type ' + meta.type + ' is not Q8_0');
        const t = this.tensorFor(meta, meta.shape[0], meta.shape[1], 1);
        return this.native.matvec(this.ctx, t, 0, asFloat32(input), 1);
    }

    matmulGeneric(meta, input) {
        if (meta.type === 8) return this.matmulQ80xF32(meta, input);
        if (this.fallbackMatmul) return this.fallbackMatmul(meta, input);
        throw new Error('Unsupported tensor type for matmul: ' + meta.type);
    }

    // One device MoE handle per layer object (src/lfm2-engine.js:129-137,
    // src/qwen3-engine.js:49-73).
    layerHandle(layer, E, K, gating, block) {
        const gt_ = gating === undefined ? GATING_SIGMOID_BIAS : gating;
        if (layer._qqMoe) {
            if (layer._qqMoe.K !== K || layer._qqMoe.gating !== gt_)
                throw new Error('MoE layer was bound with K=' + layer._qqMoe.K + ', gating=' + layer._qqMoe.gating);
            return layer._qqMoe;
        }
        if (this._gguf && block !== undefined && block !== null) {
            const p = this.native.ggufMoeParams(this._gguf, block, K, gt_);
            if (p.E !== E) throw new Error('GGUF block ' + block + ' has ' + p.E + ' experts, the layer ' + E);
            const moe = this.native.ggufMoeLayer(this.ctx, this._gguf, block, K, gt_);
            const handle = { moe: moe, H: p.H, F: p.F, E: p.E, K: p.K, gating: gt_ };
            Object.defineProperty(layer, '_qqMoe', { value: handle, enumerable: false, configurable: true });
            return handle;
        }
        const g = layer.ffnGateExps, u = layer.ffnUpExps, d = layer.ffnDownExps;
        const H = g.shape[0], F = g.shape[1];
        if (g.type !== 8 || u.type !== 8 || d.type !== 8)
            throw new Error('MoE expert tensors must be Q8_0 (type 8)');
        if (g.shape[2] !== E || d.shape[0] !== F || d.shape[1] !== H)
            throw new Error('MoE expert tensor shapes do not match [H, F, E] / [F, H, E]');
        const gt = this.tensorFor(g, H, F, E);
        const ut = this.tensorFor(u, H, F, E);
        const dt = this.tensorFor(d, F, H, E);
        const r = layer.routerWeight;
        const bias = (gt_ === GATING_SIGMOID_BIAS && layer.expProbsBias) ? readWeightF32(layer.expProbsBias, E) : null;
        const moe = this.native.moeCreate(this.ctx, r.buffer, r.offset, r.type, bias, gt, ut, dt, H, F, E, K);
        if (gt_ !== GATING_SIGMOID_BIAS) this.native.moeSetGating(this.ctx, moe, gt_);
        const handle = { moe: moe, H: H, F: F, E: E, K: K, gating: gt_ };
        Object.defineProperty(layer, '_qqMoe', { value: handle, enumerable: false, configurable: true });
        return handle;
    }

    // T tokens, each row independent (the reference runs T sequential calls,
    // src/lfm2-engine.js:550-555).  hidden is updated in place.
    moeForward(layer, X, hidden, T, opts) {
        const o = opts || {};
        const K = o.K !== undefined ? o.K : 4;
        const E = layer.ffnGateExps.shape[2];
        const h = this.layerHandle(layer, E, K, o.gating, o.block);
        let mask = null;
        if (o.mask && o.mask.size) {
            mask = new Uint8Array(h.E);
            o.mask.forEach(function (e) { if (e >= 0 && e < h.E) mask[e] = 1; });
        }
        return this.native.moeForward(this.ctx, h.moe, asFloat32(X), hidden, T, mask, !!o.wantProbs);
    }

    // Lfm2Engine._moEFFN (src/lfm2-engine.js:413-487) on `eng` (an Lfm2Engine).
    // The routing telemetry carries the same payload; it is delivered after the
    // block has run.  bufMoEOut is not written (the sum goes straight into
    // bufHidden on the device).
    moEFFN(eng, layerIdx, layer) {
        const want = !!eng.onRouterUpdate;
        const r = this.moeForward(layer, eng.bufNormed, eng.bufHidden, 1,
                                  { K: eng.nExpertsUsed, mask: eng.expertMask, wantProbs: want, block: layerIdx });
        if (want) {
            eng.onRouterUpdate({
                layer: layerIdx,
                probs: Array.from(r.probs),
                selected: Array.from(r.idx),
                weights: Array.from(r.w),
            });
        }
    }

    // Qwen3Engine._moEFFN (src/qwen3-engine.js:304-363): softmax gating, top-K
    // from the layer (layer.nExpertsUsed), same telemetry payload.
    moEFFNQwen3(eng, layerIdx, layer) {
        const want = !!eng.onRouterUpdate;
        const r = this.moeForward(layer, eng.bufNormed, eng.bufHidden, 1,
                                  { K: layer.nExpertsUsed, gating: GATING_SOFTMAX, mask: eng.expertMask,
                                    wantProbs: want, block: layerIdx });
        if (want) {
            eng.onRouterUpdate({
                layer: layerIdx,
                probs: Array.from(r.probs),
                selected: Array.from(r.idx),
                weights: Array.from(r.w),
            });
        }
    }

    release() {
        for (const e of this._lfm2) this.native.release(e.model);
        this._lfm2 = [];
        if (this._gguf) {
            this.native.release(this._gguf);
            this._gguf = null;
        }
        if (this.ctx) {
            this.native.release(this.ctx);
            this.ctx = null;
        }
    }
}

// Rebind the reference's globals (or any object holding them) to the device:
// matmulQ80xF32, matmulGeneric (type 8 here, other types to the previous
// function), Lfm2Engine.prototype._moEFFN and Qwen3Engine.prototype._moEFFN
// (each when the scope defines the class).  Throws when the device is
// unavailable; nothing is rebound in that case.
function install(scope, opts) {
    const o = opts || {};
    const dev = new MoEDevice(o.device);
    if (typeof scope.matmulGeneric === 'function') dev.fallbackMatmul = scope.matmulGeneric;
    scope.matmulQ80xF32 = function (meta, input) { return dev.matmulQ80xF32(meta, input); };
    scope.matmulGeneric = function (meta, input) { return dev.matmulGeneric(meta, input); };
    if (scope.Lfm2Engine && scope.Lfm2Engine.prototype) {
        scope.Lfm2Engine.prototype._moEFFN = function (layerIdx, layer) {
            return dev.moEFFN(this, layerIdx, layer);
        };
    }
    if (scope.Qwen3Engine && scope.Qwen3Engine.prototype) {
        scope.Qwen3Engine.prototype._moEFFN = function (layerIdx, layer) {
            return dev.moEFFNQwen3(this, layerIdx, layer);
        };
    }
    // The WebGPU engines: an engine whose buffers are this device's
    // DeviceBuffers (its _gpu is the returned device) runs _moEFFNGPU and
    // _readbackRoutingData here; any other engine keeps its own methods.
    [['Lfm2GPUEngine', GATING_SIGMOID_BIAS], ['Qwen3GPUEngine', GATING_SOFTMAX]].forEach(function (c) {
        const cls = scope[c[0]];
        if (!cls || !cls.prototype) return;
        const P = cls.prototype, block = P._moEFFNGPU, readback = P._readbackRoutingData;
        const reset = P._resetGPUState;
        if (reset) {
            P._resetGPUState = function () {
                const r = reset.apply(this, arguments);
                if (dev.ownsEngine(this)) this._qqTimeouts = dev.timeouts;
                return r;
            };
        }
        P._moEFFNGPU = function (layerIdx, gl, cl) {
            if (dev.ownsEngine(this)) return dev.moEFFNGPU(this, layerIdx, gl, cl, c[1]);
            if (block) return block.call(this, layerIdx, gl, cl);
            throw new Error(c[0] + '._moEFFNGPU: the engine\'s buffers are not on this device');
        };
        P._readbackRoutingData = function () {
            if (dev.ownsEngine(this)) return dev.readbackRoutingData(this);
            if (readback) return readback.call(this);
            return Promise.resolve();
        };
    });
    return dev;
}

module.exports = { MoEDevice: MoEDevice, DeviceBuffer: DeviceBuffer, install: install, readWeightF32: readWeightF32,
                   halfToNumber: halfToNumber, ADDON_PATH: ADDON_PATH,
                   GATING_SIGMOID_BIAS: GATING_SIGMOID_BIAS, GATING_SOFTMAX: GATING_SOFTMAX };
