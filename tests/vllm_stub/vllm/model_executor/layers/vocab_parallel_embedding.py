import torch


class VocabParallelEmbedding(torch.nn.Module):
    def __init__(self, num_embeddings, embedding_dim, params_dtype=torch.bfloat16, quant_config=None,
                 prefix=""):
        super().__init__()
        self.quant_method = quant_config.get_quant_method(self, prefix) if quant_config else None
        if self.quant_method is not None:
            self.quant_method.create_weights(self, embedding_dim, [num_embeddings], embedding_dim,
                                             num_embeddings, params_dtype)
        else:
            self.weight = torch.nn.Parameter(torch.empty(num_embeddings, embedding_dim,
                                                         dtype=params_dtype), requires_grad=False)

    def forward(self, input_):
        return self.quant_method.embedding(self, input_)


class ParallelLMHead(VocabParallelEmbedding):
    pass
