"""Writes the golden fixtures under tests/golden/*.safetensors.

The reference (KIROKOWA/ASRN, pure Python on PyTorch) is imported here, in the build container only, for the parts
of its hot path that no closed form or definition pins: the full composition of CapaASRNEstable.forward and its
gradients (asrn/estable.py:407-421), its candidate-attention stage with its gradients (estable:204-272), and its
repetition stage (estable:304-321) with the reference's own rounding order; and the same for the unprotected core
layer (asrn/nucleo.py:574-886, CapaASRN = asrn.ASRNCoreLayer). Each fixture holds only data: the
inputs, the layer's state_dict, every intermediate the hot path produces and the gradients. Nothing from the
reference itself is stored.

Run from the repository root:  python tests/golden/make_golden.py /root/reference [case names...]
"""
import json
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, layer kwargs, B, L, token range, extra settings)
CASES = [
    ('a_c16_nb4_L90', dict(chunk=16, n_bits=4), 32, 2, 90, 12, {}),
    ('b_c16_nb4_L5', dict(chunk=16, n_bits=4), 32, 1, 5, 12, {}),
    ('c_c16_nb4_L1', dict(chunk=16, n_bits=4), 32, 1, 1, 12, {}),
    ('d_default_L150', dict(), 64, 2, 150, 12, {}),
    ('e_c32_nb6_cf20_k6_shift', dict(chunk=32, n_bits=6, confirmar=20, sufijo=6), 48, 2, 200, 12,
     {'corrimiento': 2e5}),
    ('f_gamma_huge', dict(chunk=16, n_bits=3), 32, 1, 96, 7, {'gamma_fill': 1e9}),
    ('g_default_V6_L300', dict(), 32, 2, 300, 6, {}),
    ('h_streak_exact', dict(chunk=16, n_bits=4), 32, 2, 120, 5, {'kappa_r_zero': True}),
    # group-B protections (estable:72-77): the gate's tanh cap (logits pushed well past it) and the kappa floor
    # (two Hawkes rates and the streak rate pushed below it)
    ('i_textos_largos', dict(chunk=16, n_bits=4), 32, 2, 120, 12, {'prot': 'textos_largos', 'largo': 1024}),
    # bf16 autocast on the CPU (the reference's own bf16 case, tests/test_nucleo.py:476: d 64, default tables,
    # B 2, L 160): the layer and its stages under torch.autocast('cpu', bfloat16), and the fp32 layer beside it
    ('j_bf16_d64_L160', dict(), 64, 2, 160, 12, {'autocast': 'bf16'}),
    # the unprotected core layer (asrn.ASRNCoreLayer = nucleo.CapaASRN, v89 numerics: the fp32 clock with the score's
    # clock term formed as (log alfa_k + rate B_k) - rate B_q, the -1e9 fill instead of the exact mask, no clamps) on
    # ordinary inputs, and with gamma = 1e9, where every valid score of a query sinks below -1e9 and the fill leaks
    # weight to invalid keys (the case the protected layer exists for, estable:20-24)
    ('k_nucleo_d64_L150', dict(), 64, 2, 150, 12, {'clase': 'nucleo'}),
    ('l_nucleo_c16_nb4_L120', dict(chunk=16, n_bits=4), 32, 2, 120, 9, {'clase': 'nucleo'}),
    ('m_nucleo_gamma_huge', dict(chunk=16, n_bits=3), 32, 1, 96, 7, {'clase': 'nucleo', 'gamma_fill': 1e9}),
    # the candidate stage with the clock moved by a constant (acc.Bt = Bt + 4e5): only clock differences enter the
    # scores, but the core layer's fp32 form (log alfa_k + rate B_k) - rate B_q rounds at ulp(rate B) ~ 1e-3 there,
    # which tells it apart from the difference form
    ('n_nucleo_reloj_desplazado', dict(chunk=16, n_bits=4), 32, 2, 120, 9, {'clase': 'nucleo', 'reloj_extra': 4e5}),
]


def build(ref_root, only=()):
    sys.path.insert(0, ref_root)
    os.environ['ASRN_TRITON'] = '0'             # the reference's PyTorch path (the CPU has no Triton kernels anyway)
    import contextlib

    import asrn.estable as est
    import asrn.nucleo as v89

    for name, kw, d, B, L, V, extra in CASES:
        if only and name not in only:
            continue
        torch.manual_seed(0)
        prot = est.Protecciones.textos_largos(extra['largo']) if extra.get('prot') == 'textos_largos' else None
        if extra.get('clase') == 'nucleo':
            capa = v89.CapaASRN(d, **kw)
        else:
            capa = est.CapaASRNEstable(d, protecciones=prot, **kw)
        with torch.no_grad():
            g = torch.Generator().manual_seed(1)
            for n, p in capa.named_parameters():
                p.add_(torch.randn(p.shape, generator=g) * (0.5 if n in v89._NUEVOS_V87 else 0.05))
            capa.gamma.abs_()
            if 'corrimiento' in extra:
                capa.b_reloj[0] += extra['corrimiento']
            if 'gamma_fill' in extra:
                capa.gamma.fill_(extra['gamma_fill'])
            if extra.get('kappa_r_zero'):
                capa.log_kappa_racha.fill_(-200.0)
            if extra.get('prot') == 'textos_largos':
                capa.g.weight.mul_(100.0)
                capa.log_kappa[2:] = -12.0
                capa.log_kappa_racha.fill_(-12.0)
        bf16 = extra.get('autocast') == 'bf16'
        autocast = (lambda: torch.autocast('cpu', dtype=torch.bfloat16)) if bf16 else contextlib.nullcontext
        gx = torch.Generator().manual_seed(2)
        x = torch.randint(0, V, (B, L), generator=gx)
        x[:, L // 2:L // 2 + L // 4] = x[:, :L // 4].clone()
        E0 = torch.randn(V, d, generator=gx)[x].contiguous()
        h0 = torch.randn(B, L, d, generator=gx)
        gy = torch.randn(B, L, d, generator=torch.Generator().manual_seed(3))
        out = {'x': x, 'E': E0, 'h': h0, 'gy': gy}
        for k, v in capa.state_dict().items():
            out['p.' + k] = v.clone()

        # whole layer forward + backward (under autocast for a bf16 case, and then also in fp32 with suffix 32)
        for suffix, ctx in (('', autocast),) + ((('32', contextlib.nullcontext),) if bf16 else ()):
            E, h = E0.clone().requires_grad_(), h0.clone().requires_grad_()
            capa.zero_grad()
            with ctx():
                y = capa(E, h, x)
            (y.float() * gy).sum().backward()
            out['y' + suffix] = y.detach().float()
            out['gE' + suffix] = E.grad
            out['gh' + suffix] = h.grad
            for n, p in capa.named_parameters():
                if p.grad is not None:
                    out['g' + suffix + '.' + n] = p.grad.clone()

        # stage outputs, forward only
        with torch.no_grad(), autocast():
            sig = v89.firmas_de_piezas(x)
            Qc, Kc, beta, la = capa._contexto(h0)
            Bt = beta.cumsum(1)
            phi, Vv = capa._phi_y_valores(E0)
            T = capa.n_tablas
            ids = capa._ids(phi).transpose(1, 2).reshape(B * T, L)
            orden = ids.argsort(dim=-1, stable=True)
            claves = capa._claves_vistos(sig)
            ok, rep = capa._ordenar_claves(claves)
        out.update(sig=sig, Qc=Qc, Kc=Kc, beta=beta, log_alfa=la, Bt=Bt, phi=phi, V=Vv, ids=ids,
                   orden=orden, claves=claves, orden_k=ok, repetido=rep.to(torch.uint8))

        # candidate stage with its own gradients: phi and V enter as leaves (the clock moved by reloj_extra when given,
        # kept as acc.Bt)
        Bt_acc = Bt + extra['reloj_extra'] if 'reloj_extra' in extra else Bt
        if 'reloj_extra' in extra:
            out['acc.Bt'] = Bt_acc
        leaves = {k: t.clone().requires_grad_() for k, t in
                  dict(phi=phi, V=Vv, Qc=Qc, Kc=Kc, Bt=Bt_acc, log_alfa=la).items()}
        orig = capa._phi_y_valores
        capa._phi_y_valores = lambda _E: (leaves['phi'], leaves['V'])
        capa.zero_grad()
        with autocast():
            acc = capa._acumular(E0, leaves['Qc'], leaves['Kc'], leaves['Bt'], leaves['log_alfa'], sig)
        capa._phi_y_valores = orig
        gs = torch.randn(B, L, d, generator=torch.Generator().manual_seed(4))
        (acc['salida'].float() * gs).sum().backward()
        out['acc.gs'] = gs
        for k in ('salida', 'peso_total', 'mejor', 'pico', 'peso_ctx'):
            out['acc.' + k] = acc[k].detach()
        for k, t in leaves.items():
            out['acc.g_' + k] = t.grad if t.grad is not None else torch.zeros_like(t)
        out['acc.g_w_sufijo'] = capa.w_sufijo.grad.clone()
        out['acc.g_gamma'] = capa.gamma.grad.clone()

        # repetition stage with its own gradients
        rl = {k: t.clone().requires_grad_() for k, t in dict(beta=beta, Bt=Bt, log_alfa=la).items()}
        capa.zero_grad()
        r = capa._repeticion(sig, rl['beta'], rl['Bt'], rl['log_alfa'])
        gh_ = torch.randn(B, L, capa.vistos, generator=torch.Generator().manual_seed(5))
        gr_ = torch.randn(B, L, generator=torch.Generator().manual_seed(6))
        ((r['hawkes'] * gh_).sum() + (r['racha'] * gr_).sum()).backward()
        out['rep.gh'] = gh_
        out['rep.gr'] = gr_
        for k in ('vistos', 'hawkes', 'racha'):
            out['rep.' + k] = r[k].detach()
        for k, t in rl.items():
            out['rep.g_' + k] = t.grad if t.grad is not None else torch.zeros_like(t)
        out['rep.g_log_kappa'] = capa.log_kappa.grad.clone()
        out['rep.g_log_kappa_racha'] = capa.log_kappa_racha.grad.clone()

        out = {k: v.contiguous() for k, v in out.items()}
        meta = {'d': str(d), 'B': str(B), 'L': str(L), 'V': str(V), 'kw': json.dumps(kw), 'extra': json.dumps(extra)}
        save_file(out, os.path.join(HERE, name + '.safetensors'), metadata=meta)
        print(name, sum(v.numel() * v.element_size() for v in out.values()) // 1024, 'KiB')


if __name__ == '__main__':
    build(sys.argv[1] if len(sys.argv) > 1 else '/root/reference', tuple(sys.argv[2:]))
