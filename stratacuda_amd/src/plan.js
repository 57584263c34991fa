// The decoder as data. buildProgram(g) lists, once per model geometry, every
// kernel-level instruction of a token's pass through the network: the
// embedding, each layer (PLE when the layer carries it, the attention-side
// stream mix, the gated-delta-rule or attention mixer, the write-back, the
// FFN-side mix, the routed MoE, the write-back) and the output head. One
// interpreter (interpreter.js) executes the same instruction lists for a
// decode step (one token, the reference's one-token kernels) and for a
// prompt chunk (n tokens, its *_batch kernels), so the two paths cannot
// drift apart.
//
// Every instruction is a plain object: `op` names the handler, register
// names (strings) name its inputs and outputs, and `weights` maps each
// parameter to [tensor name, expected shape]. The shape gate of a session
// (weightShapes) is read off the program itself, so a tensor is checked
// exactly when some instruction reads it. Register values are per token:
// a register of length L holds n * L values in an n-token chunk, and the
// `rows` of a norm or slice count rows per token.
//
// The launch order inside each list, the scalar arguments and which buffer
// feeds which parameter are the reference's (src/engine.js:76-156,
// src/prefill.js:14-78): every f32 rounding of the model depends on them.

// Register holding the residual streams of the tokens in flight.
export const RESIDUAL = '$residual';

// One-token and token-batch kernel of each instruction that has both.
export const KERNELS = {
    hcMix: ['strata_hc_mix', 'strata_hc_mix_batch'],
    hcWrite: ['strata_hc_write', 'strata_hc_write_batch'],
    conv: ['strata_conv', 'strata_conv_batch'],
    gdnGates: ['strata_gdn_gates', 'strata_gdn_gates_batch'],
    gdnScan: ['strata_gdn_step', 'strata_gdn_batch'],
    kvAppend: ['strata_kv_append', 'strata_kv_append_batch'],
    attention: ['strata_attention', 'strata_attention_batch'],
    attentionGate: ['strata_attention_gate', 'strata_attention_gate_batch'],
    pleBroadcast: ['strata_ple_broadcast', 'strata_ple_broadcast_batch'],
    router: ['strata_router', 'strata_router_batch'],
    combine: ['strata_moe_combine', 'strata_moe_combine_batch'],
};

const isAttentionLayer = (g, layer) => layer % g.qsaInterval === g.qsaInterval - 1;

// The hyper-connection read of the residual streams into one mixer input
// (src/engine.js:76-83): per-stream RMSNorm, a rank-`g.rank` gate and the
// stream mix; `inject` adds the per-stream write-back weights.
function streamMix(g, prefix, out, inject) {
    const hc = g.width * g.streams, r = name => out + '.' + name;
    const list = [
        {op: 'norm', x: RESIDUAL, y: r('norm'), cols: g.width, rows: g.streams, weightRows: g.streams,
            weights: {W: [prefix + 'norm.weight', [hc]]}},
        {op: 'project', x: r('norm'), y: r('down'), weights: {W: [prefix + 'down.weight', [hc, g.rank]]}},
        {op: 'elementwise', a: r('down'), b: r('down'), y: r('low'), mode: 1, scale: 1 / g.streams},
        {op: 'project', x: r('low'), y: r('gate'), weights: {W: [prefix + 'up.weight', [g.rank, hc]]}},
        {op: 'hcMix', norm: r('norm'), gate: r('gate'), y: out},
    ];
    if (inject) list.push({op: 'project', x: r('norm'), y: r('inject'),
        weights: {W: [prefix + 'inject.weight', [hc, g.streams]]}});
    return list;
}

// Per-layer embedding block (src/engine.js:86-96): n-gram rows, a key/query
// gate per stream, a dilated causal convolution over the gated rows, added
// into the residual.
function pleBlock(g) {
    const p = 'blk.' + g.pleLayer + '.ple_', hc = g.width * g.streams;
    const vec = (name, shape) => ({W: [p + name, shape]});
    return [
        {op: 'pleRows', y: 'ple.rows'},
        {op: 'project', x: 'ple.rows', y: 'ple.rawKey', weights: vec('key.weight', [g.width, hc])},
        {op: 'norm', x: 'ple.rawKey', y: 'ple.key', cols: g.width, rows: g.streams, weightRows: g.streams,
            weights: vec('norm_key.weight', [hc])},
        {op: 'norm', x: RESIDUAL, y: 'ple.query', cols: g.width, rows: g.streams, weightRows: g.streams,
            weights: vec('norm_query.weight', [hc])},
        {op: 'project', x: 'ple.rows', y: 'ple.value', weights: vec('value.weight', [g.width, g.width])},
        {op: 'pleGate', key: 'ple.key', query: 'ple.query', y: 'ple.gate'},
        {op: 'pleBroadcast', value: 'ple.value', gate: 'ple.gate', y: 'ple.gated'},
        {op: 'norm', x: 'ple.gated', y: 'ple.normed', cols: g.width, rows: g.streams, weightRows: g.streams,
            weights: vec('norm_conv.weight', [hc])},
        {op: 'conv', x: 'ple.normed', y: 'ple.conv', history: 'pleHistory', channels: hc, taps: g.pleTaps,
            dilation: g.pleDilation, weights: vec('conv1d.weight', [g.pleTaps, hc])},
        {op: 'pleAdd', gated: 'ple.gated', conv: 'ple.conv'},
    ];
}

// Gated delta-rule mixer (src/engine.js:97-111).
function deltaRule(g, layer, x, out) {
    const p = 'blk.' + layer + '.', qk = g.ssmDim * g.keyHeads, vn = g.ssmDim * g.valueHeads, c = 2 * qk + vn;
    const w = (name, shape) => ({W: [p + name, shape]});
    return [
        {op: 'project', x, y: 'gdn.qkv', weights: w('attn_qkv.weight', [g.width, c])},
        {op: 'conv', x: 'gdn.qkv', y: 'gdn.conv', history: 'conv', channels: c, taps: 4, dilation: 1,
            weights: w('ssm_conv1d.weight', [4, c])},
        {op: 'slice', x: 'gdn.conv', y: 'gdn.qRaw', width: qk, rows: 1, stride: c, offset: 0},
        {op: 'slice', x: 'gdn.conv', y: 'gdn.kRaw', width: qk, rows: 1, stride: c, offset: qk},
        {op: 'slice', x: 'gdn.conv', y: 'gdn.v', width: vn, rows: 1, stride: c, offset: 2 * qk},
        {op: 'norm', x: 'gdn.qRaw', y: 'gdn.q', cols: g.ssmDim, rows: g.keyHeads, weightRows: 1, mode: 1,
            scale: 1 / Math.sqrt(g.ssmDim)},
        {op: 'norm', x: 'gdn.kRaw', y: 'gdn.k', cols: g.ssmDim, rows: g.keyHeads, weightRows: 1, mode: 1},
        {op: 'project', x, y: 'gdn.alpha', weights: w('ssm_alpha.weight', [g.width, g.valueHeads])},
        {op: 'project', x, y: 'gdn.beta', weights: w('ssm_beta.weight', [g.width, g.valueHeads])},
        {op: 'gdnGates', alpha: 'gdn.alpha', beta: 'gdn.beta', decay: 'gdn.decay', strength: 'gdn.strength',
            weights: {A: [p + 'ssm_a', [g.valueHeads]], Dt: [p + 'ssm_dt.bias', [g.valueHeads]]}},
        {op: 'gdnScan', q: 'gdn.q', k: 'gdn.k', v: 'gdn.v', decay: 'gdn.decay', strength: 'gdn.strength', y: 'gdn.y'},
        {op: 'project', x, y: 'gdn.z', weights: w('attn_gate.weight', [g.width, vn])},
        {op: 'norm', x: 'gdn.y', y: 'gdn.yNorm', cols: g.ssmDim, rows: g.valueHeads, weightRows: 1,
            weights: w('ssm_norm.weight', [g.ssmDim])},
        {op: 'elementwise', a: 'gdn.yNorm', b: 'gdn.z', y: 'gdn.gated', mode: 4},
        {op: 'project', x: 'gdn.gated', y: out, weights: w('ssm_out.weight', [vn, g.width])},
    ];
}

// Gated attention mixer over the session's KV cache (src/engine.js:115-124).
function attention(g, layer, x, out) {
    const p = 'blk.' + layer + '.', hd = g.headDim, kv = g.kvHeads * hd;
    const w = (name, shape) => ({W: [p + name, shape]});
    return [
        {op: 'project', x, y: 'qsa.full', weights: w('attn_q.weight', [g.width, 2 * g.heads * hd])},
        {op: 'slice', x: 'qsa.full', y: 'qsa.qRaw', width: hd, rows: g.heads, stride: 2 * hd, offset: 0},
        {op: 'norm', x: 'qsa.qRaw', y: 'qsa.qNorm', cols: hd, rows: g.heads, weightRows: 1,
            weights: w('attn_q_norm.weight', [hd])},
        {op: 'rope', x: 'qsa.qNorm', y: 'qsa.q', heads: g.heads},
        {op: 'project', x, y: 'qsa.kRaw', weights: w('attn_k.weight', [g.width, kv])},
        {op: 'norm', x: 'qsa.kRaw', y: 'qsa.kNorm', cols: hd, rows: g.kvHeads, weightRows: 1,
            weights: w('attn_k_norm.weight', [hd])},
        {op: 'rope', x: 'qsa.kNorm', y: 'qsa.k', heads: g.kvHeads},
        {op: 'project', x, y: 'qsa.v', weights: w('attn_v.weight', [g.width, kv])},
        {op: 'kvAppend', k: 'qsa.k', v: 'qsa.v', width: kv},
        {op: 'attention', q: 'qsa.q', y: 'qsa.att'},
        {op: 'attentionGate', attention: 'qsa.att', full: 'qsa.full', y: 'qsa.gated'},
        {op: 'project', x: 'qsa.gated', y: out, weights: w('attn_output.weight', [g.heads * hd, g.width])},
    ];
}

// Routed experts plus the shared expert (src/engine.js:125-156). The MoE
// instruction reads every expert's three projections (f32 stores) or the
// layer's packed blobs (Q2 stores; the gate still checks the f32 names the
// manifest describes).
function routedExperts(g, layer, x, out) {
    const p = 'blk.' + layer + '.', weights = {
        router: [p + 'ffn_gate_inp.weight', [g.width, g.experts]],
        sharedGate: [p + 'ffn_gate_inp_shexp.weight', [g.width]],
    };
    for (const role of ['gate', 'up', 'down']) {
        const shape = role === 'down' ? [g.ff, g.width] : [g.width, g.ff];
        weights['shared.' + role] = [p + 'ffn_' + role + '_shexp.weight', shape];
        for (let e = 0; e < g.experts; e++) weights[e + '.' + role] = [p + 'expert.' + e + '.' + role, shape];
    }
    return [{op: 'moe', layer, x, y: out, weights}];
}

// The whole decoder: {embed, layers[l], head} instruction lists.
export function buildProgram(g) {
    const layers = [];
    for (let l = 0; l < g.layers; l++) {
        const p = 'blk.' + l + '.', list = [];
        if (l === g.pleLayer) list.push(...pleBlock(g));
        list.push(...streamMix(g, p + 'hc_attn_', 'attn', true));
        list.push(...(isAttentionLayer(g, l) ? attention(g, l, 'attn', 'mixer') : deltaRule(g, l, 'attn', 'mixer')));
        list.push({op: 'hcWrite', x: 'mixer', inject: 'attn.inject'});
        list.push(...streamMix(g, p + 'hc_ffn_', 'ffn', true));
        list.push(...routedExperts(g, l, 'ffn', 'experts'));
        list.push({op: 'hcWrite', x: 'experts', inject: 'ffn.inject'});
        layers.push({index: l, attention: isAttentionLayer(g, l), list});
    }
    return {
        embed: [{op: 'embed', weights: {table: ['token_embd.weight', [g.width, g.vocab]]}}],
        layers,
        head: [...streamMix(g, 'output_hc_', 'head', false),
            {op: 'project', x: 'head', y: 'logits', weights: {W: ['output.weight', [g.width, g.vocab]]}},
            {op: 'argmax', x: 'logits', y: 'next'}],
    };
}

// Every [tensor name, shape] the program reads, each name once, in program
// order.
export function weightShapes(program) {
    const seen = new Map();
    const visit = list => {
        for (const ins of list)
            for (const [name, shape] of Object.values(ins.weights || {}))
                if (!seen.has(name)) seen.set(name, shape);
    };
    visit(program.embed);
    for (const layer of program.layers) visit(layer.list);
    visit(program.head);
    return Array.from(seen);
}

// The recurrent state one layer keeps across tokens, by kind of mixer:
// attention layers a KV cache of `context` positions, delta-rule layers the
// [value heads x dim x dim] state and the last three convolution inputs.
export function layerStateShapes(g, layer) {
    if (isAttentionLayer(g, layer))
        return {keys: g.context * g.kvHeads * g.headDim, values: g.context * g.kvHeads * g.headDim};
    const c = (2 * g.keyHeads + g.valueHeads) * g.ssmDim;
    return {ssm: g.ssmDim * g.valueHeads * g.ssmDim, conv: c * 3};
}
