'use strict';
/**
 * Drives the Node host (webllm_amd/js) for tests/test_node_host.py.
 *
 *   node node_host_check.js abi <dir>   no GPU: addon exports, plans, validation codes, parse of
 *                                       <dir>/model.safetensors; prints one JSON line
 *   node node_host_check.js gpu <dir>   loads <dir>/model.safetensors with loadQwenWeights and
 *                                       runs the cases of <dir>/cases.json, writing each output
 *                                       to <dir>/<out>; prints one JSON line
 * Correctness is judged by the Python side against the C oracle.
 */
const fs = require('fs');
const path = require('path');
const q = require('../../webllm_amd/js');

function readF32(file) {
    const b = fs.readFileSync(file);
    return new Float32Array(b.buffer.slice(b.byteOffset, b.byteOffset + b.byteLength));
}

function writeTyped(file, typed) {
    fs.writeFileSync(file, Buffer.from(typed.buffer, typed.byteOffset, typed.byteLength));
}

function abi(dir) {
    const plans = [[1, 4864, 896], [4, 896, 4864], [16, 128, 896], [64, 896, 896], [1, 13, 20]]
        .map(([M, N, K]) => Object.assign({ M, N, K }, q.addon.planLinear(M, N, K, 128)));
    const desc = (K, N, group, bits) => q.makeDesc(0, null, 0, K, N, group, null, bits);
    const validate = {
        ok: q.addon.validate(desc(896, 128, 128, 4), 1 << 30),
        bits: q.addon.validate(desc(896, 128, 128, 3), 1 << 30),
        group: q.addon.validate(desc(896, 128, 0, 4), 1 << 30),
        dims: q.addon.validate(desc(0, 128, 128, 4), 1 << 30),
        pack: q.addon.validate(desc(896, 128, 100, 4), 1 << 30),
    };
    const file = q.parseSafetensors(fs.readFileSync(path.join(dir, 'model.safetensors')));
    let badParse = null;
    try { q.parseSafetensors(new Uint8Array(4)); } catch (e) { badParse = e.message; }
    // the loader's format probes (qwen-format.ts:112-130) and readF16Rows (qwen-loader.ts:70-93)
    const probes = { gIdxOk: null, gIdxActOrder: null, urls: [], badUrl: null };
    try { q.checkGIdx(file, 'model.layers.1.mlp.gate_proj', 256, 128); } catch (e) { probes.gIdxOk = e.message; }
    const act = path.join(dir, 'act_order.safetensors');
    if (fs.existsSync(act)) {
        const f2 = q.parseSafetensors(fs.readFileSync(act));
        try { q.checkGIdx(f2, 'model.layers.1.mlp.gate_proj', 256, 128); } catch (e) { probes.gIdxActOrder = e.message; }
    }
    writeTyped(path.join(dir, 'rows.f32'), q.readF16Rows(file, 'model.embed_tokens.weight', 5, 3, 256));
    probes.zerosK = q.countStoredZeros(q.readTensorBytes(file, 'model.layers.0.self_attn.k_proj.qzeros'), 2, 128,
        new Array(16).fill(0));
    probes.urls = [q.urlToPath('file:///tmp/a%20b/model.safetensors'), q.urlToPath('rel/model.safetensors')];
    try { q.urlToPath('https://huggingface.co/m/model.safetensors'); } catch (e) { probes.badUrl = e.message; }
    console.log(JSON.stringify({
        exports: Object.keys(q.addon).sort(),
        plans,
        validate,
        sizes: q.addon.gptqSizes(896, 4864, 128),
        tensors: Object.keys(file.header).length,
        embedShape: q.requireTensor(file, 'model.embed_tokens.weight').shape,
        badParse,
        probes,
    }));
}

async function gpu(dir) {
    const spec = JSON.parse(fs.readFileSync(path.join(dir, 'cases.json'), 'utf8'));
    const ctx = new q.Context(0);
    try {
        const model = new q.QuantLinearModel(ctx, 64 << 20);
        const progress = [];
        const pending = q.loadQwenWeights(ctx, model, {
            url: 'file://' + path.join(dir, 'model.safetensors'), config: spec.config, keepLayer: 0,
            keepEmbedRows: { start: 100, rows: 4 }, onProgress: (i, n) => progress.push(i),
        });
        const isPromise = pending instanceof Promise;
        const res = await pending;
        writeTyped(path.join(dir, 'kept_qW.f32'), res.layer.qW);
        writeTyped(path.join(dir, 'embed_rows.f32'), res.embedRows);
        // an act-order (desc_act) checkpoint is rejected (qwen-format.ts:125-130)
        let actOrder = null;
        const m2 = new q.QuantLinearModel(ctx, 64 << 20);
        try {
            await q.loadQwenWeights(ctx, m2, { path: path.join(dir, 'act_order.safetensors'), config: spec.config });
        } catch (e) { actOrder = e.message; }
        m2.release();
        const pool = new q.ActivationArena(ctx, 32 << 20);
        for (const c of spec.gemm) {
            const A = pool.alloc([c.M, c.K], c.f16 ? 'f16' : 'f32');
            A.write(Uint8Array.from(fs.readFileSync(path.join(dir, c.x))));  // f32 or f16 bits
            const C = pool.alloc([c.M, c.N]);
            model.gemm(A, c.weight, C, c.bias, c.M, c.N, c.K);
            ctx.sync();
            writeTyped(path.join(dir, c.out), C.read());
            pool.reset();
        }
        for (const b of spec.batch) {
            const A = pool.alloc([b.M, b.K]);
            A.write(readF32(path.join(dir, b.x)));
            const Cs = b.weights.map((w, i) => pool.alloc([b.M, b.N[i]]));
            model.gemmBatch(A, b.weights, Cs, b.M);
            ctx.sync();
            Cs.forEach((C, i) => writeTyped(path.join(dir, b.outs[i]), C.read()));
            pool.reset();
        }
        // a chained sequence run from JavaScript: each linear reads the previous one's output
        if (spec.seq) {
            const sq = spec.seq;
            const descs = sq.weights.map((w) => model.linear(w).desc);
            const X = pool.alloc([sq.M, descs[0].K]);
            X.write(readF32(path.join(dir, sq.x)));
            const Ys = descs.map((d) => pool.alloc([sq.M, d.N]));
            const xOffs = descs.map((d, i) => (i === 0 ? X.offset : Ys[i - 1].offset));
            const seq = ctx.seq(descs, model.weights, pool.arena, xOffs, q.QL_DTYPE_F32, sq.M,
                Ys.map((y) => y.offset));
            const info = seq.info;
            seq.run();
            seq.status();
            Ys.forEach((Y, i) => writeTyped(path.join(dir, sq.outs[i]), Y.read()));
            seq.destroy();
            pool.reset();
            spec.seqInfo = info;
        }
        // a fused layer run from JavaScript (ql_seq_create_fused): q/k/v <- rmsnorm(h, inNorm),
        // h1 = h + o(q), gate/up <- rmsnorm(h1, postNorm), h2 = h1 + down(silu(gate) * up)
        if (spec.fused) {
            const fz = spec.fused;
            const names = ['qW', 'kW', 'vW', 'oW', 'gateW', 'upW', 'downW'];
            const descs = names.map((k) => model.linear(`L0.${k}`).desc);
            const H = pool.alloc([fz.M, descs[0].K]);
            H.write(readF32(path.join(dir, fz.x)));
            const Y = descs.map((d) => pool.alloc([fz.M, d.N]));
            const ln1 = model.f32Weights.get('L0.inNorm').offset;
            const ln2 = model.f32Weights.get('L0.postNorm').offset;
            const norm = (off) => ({ normWOff: off, normEps: fz.eps });
            const xOffs = [H, H, H, Y[0], Y[3], Y[3], Y[4]].map((t) => t.offset);
            const fuse = [norm(ln1), norm(ln1), norm(ln1), { resOff: H.offset }, norm(ln2), norm(ln2),
                { x2Off: Y[5].offset, resOff: Y[3].offset }];
            const seq = ctx.seq(descs, model.weights, pool.arena, xOffs, q.QL_DTYPE_F32, fz.M,
                Y.map((y) => y.offset), fuse);
            spec.fusedInfo = seq.info;
            seq.run();
            seq.status();
            Y.forEach((y, i) => writeTyped(path.join(dir, fz.outs[i]), y.read()));
            seq.destroy();
            pool.reset();
            // both fused operands at once are refused (norm and x2 exclude each other)
            try {
                ctx.seq([descs[0]], model.weights, pool.arena, [H.offset], q.QL_DTYPE_F32, fz.M, [Y[0].offset],
                    [{ normWOff: ln1, x2Off: Y[5].offset }]);
            } catch (e) { spec.fusedBoth = e.message; }
        }
        const u = spec.unpack;
        const U = pool.alloc([u.N, u.K], 'f16');
        model.unpackF16(u.weight, U);
        ctx.sync();
        writeTyped(path.join(dir, u.out), U.read());
        pool.reset();
        // the batched form over several weights at once
        const ua = spec.unpackAll;
        const UA = ua.weights.map((w, i) => pool.alloc([ua.N[i], ua.K[i]], 'f16'));
        model.unpackAllF16(ua.weights, UA);
        ctx.sync();
        UA.forEach((t, i) => writeTyped(path.join(dir, ua.outs[i]), t.read()));
        pool.reset();

        // dequantizeGptqInt4 with the reference's params object, from the parsed file
        const file = q.parseSafetensors(fs.readFileSync(path.join(dir, 'model.safetensors')));
        const d = spec.dequant;
        const W = q.dequantizeGptqInt4({
            qweight: q.readTensorBytes(file, `${d.prefix}.qweight`),
            qzeros: q.readTensorBytes(file, `${d.prefix}.qzeros`),
            scales: q.readTensorF32(file, `${d.prefix}.scales`),
            inFeatures: d.K, outFeatures: d.N, groupSize: 128,
        }, ctx);
        writeTyped(path.join(dir, d.out), W);
        // any Float32Array scales (quant.ts:22-23): not fp16 values, tiny, huge
        const ds = spec.dequantF32;
        const W2 = q.dequantizeGptqInt4({
            qweight: Uint8Array.from(fs.readFileSync(path.join(dir, ds.qweight))),
            qzeros: Uint8Array.from(fs.readFileSync(path.join(dir, ds.qzeros))),
            scales: readF32(path.join(dir, ds.scales)),
            inFeatures: ds.K, outFeatures: ds.N, groupSize: ds.group,
        }, ctx);
        writeTyped(path.join(dir, ds.out), W2);

        // residual add + RMSNorm, SiLU-mul, and the KV cache with decode attention
        const el = spec.elem;
        const rd = (f) => Uint8Array.from(fs.readFileSync(path.join(dir, f)));
        const EX = pool.alloc([el.M, el.C]), ER = pool.alloc([el.M, el.C]);
        const ES = pool.alloc([el.M, el.C]), EY = pool.alloc([el.M, el.C]);
        EX.write(rd(el.x));
        ER.write(rd(el.r));
        model.rmsnorm(EX, 'L0.inNorm', EY, el.M, el.C, 1e-6, ER, ES);
        const EG = pool.alloc([el.n]), EU = pool.alloc([el.n]), EO = pool.alloc([el.n]);
        EG.write(rd(el.g));
        EU.write(rd(el.u));
        model.siluMul(EG, EU, EO, el.n);
        ctx.sync();
        writeTyped(path.join(dir, 'el_y.f32'), EY.read());
        writeTyped(path.join(dir, 'el_s.f32'), ES.read());
        writeTyped(path.join(dir, 'el_o.f32'), EO.read());
        pool.reset();
        const kv = new q.KvCache(ctx, spec.config);
        for (let t = 0; t < spec.kvSteps; t++) {
            const K = pool.alloc([1, kv.rowLen]), V = pool.alloc([1, kv.rowLen]);
            const Q = pool.alloc([1, spec.config.nEmbd]), O = pool.alloc([1, spec.config.nEmbd]);
            K.write(rd(`kv_k${t}`));
            V.write(rd(`kv_v${t}`));
            Q.write(rd(`kv_q${t}`));
            kv.store(1, K, V, 1, t);
            kv.attend(1, Q, O, 1, t);
            ctx.sync();
            writeTyped(path.join(dir, `kv_o${t}.f32`), O.read());
            pool.reset();
        }
        kv.release();

        const errors = {};
        const expectThrow = (key, fn) => {
            try { fn(); errors[key] = null; } catch (e) { errors[key] = e.message; }
        };
        const A = pool.alloc([1, spec.config.nEmbd]);
        const C = pool.alloc([1, spec.config.nEmbd]);
        expectThrow('missingWeight', () => model.gemm(A, 'L9.qW', C, null, 1, spec.config.nEmbd, spec.config.nEmbd));
        expectThrow('wrongShape', () => model.gemm(A, 'L0.qW', C, null, 1, spec.config.nEmbd + 8, spec.config.nEmbd));
        expectThrow('missingBias', () => model.gemm(A, 'L0.oW', C, 'L0.oB', 1, spec.config.nEmbd, spec.config.nEmbd));
        expectThrow('duplicate', () => model.uploadF32('finalNorm', new Float32Array(4)));
        expectThrow('bits', () => q.dequantizeGptqInt4({ qweight: new Uint8Array(4), scales: new Float32Array(1), inFeatures: 8, outFeatures: 1, bits: 8 }, ctx));
        // tensors of another ActivationArena are refused before any launch
        const other = new q.ActivationArena(ctx, 1 << 20);
        const Y2 = other.alloc([1, spec.config.nEmbd]);
        expectThrow('rmsnormArena', () => model.rmsnorm(A, 'L0.inNorm', Y2, 1, spec.config.nEmbd, 1e-6));
        expectThrow('rmsnormSumArena', () => model.rmsnorm(A, 'L0.inNorm', C, 1, spec.config.nEmbd, 1e-6, null, Y2));
        const kv2 = new q.KvCache(ctx, spec.config);
        expectThrow('attendArena', () => kv2.attend(0, A, Y2, 1, 0));
        kv2.release();
        other.release();
        pool.release();
        model.release();
        console.log(JSON.stringify({
            device: ctx.info(), tensorCount: res.tensorCount, gpuBytes: res.gpuBytes,
            fileBytes: res.fileBytes, progress, errors, seqInfo: spec.seqInfo || null,
            fusedInfo: spec.fusedInfo || null, fusedBoth: spec.fusedBoth || null,
            isPromise, storedZeros: res.storedZeros, actOrder,
        }));
    } finally {
        ctx.destroy();
    }
}

const [mode, dir] = process.argv.slice(2);
if (mode === 'abi') abi(dir);
else if (mode === 'gpu') gpu(dir).catch((e) => { console.error(e && e.stack ? e.stack : e); process.exit(1); });
else { console.error('usage: node node_host_check.js abi|gpu <dir>'); process.exit(2); }
